// Runs one gpa_decode_step of the host build on a problem dump (test
// infrastructure).  Dump: struct bytes; the buffers (each allocated here with
// its exact size, so AddressSanitizer bounds every access); the pointer fields
// as (struct offset, buffer, byte offset).  Writes every buffer back.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "gpa_hip.h"

thread_local EmuIdx threadIdx, blockIdx;
std::barrier<>* emu_block_barrier;
std::vector<std::unique_ptr<std::barrier<>>> emu_wave_barrier;
float emu_xchg[16][64];
static std::string last_error;
int fail(int code, const char* message) {
  last_error = message;
  return code;
}
int check_launch(const char*) { return 0; }

static int64_t get(FILE* f) {
  int64_t x = 0;
  if (fread(&x, 8, 1, f) != 1) exit(4);
  return x;
}

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 2;
  std::vector<char> st(get(f));
  if (fread(st.data(), 1, st.size(), f) != st.size()) return 4;
  const int64_t nbuf = get(f);
  std::vector<char*> buf(nbuf);
  std::vector<int64_t> bytes(nbuf);
  for (int64_t i = 0; i < nbuf; ++i) {
    bytes[i] = get(f);
    buf[i] = static_cast<char*>(malloc(bytes[i]));
    if (fread(buf[i], 1, bytes[i], f) != (size_t)bytes[i]) return 4;
  }
  const int64_t nptr = get(f);
  for (int64_t i = 0; i < nptr; ++i) {
    const int64_t off = get(f), id = get(f), boff = get(f);
    char* p = buf[id] + boff;
    memcpy(st.data() + off, &p, 8);
  }
  fclose(f);
  const int rc = gpa_decode_step(reinterpret_cast<gpa_decode_problem*>(st.data()), nullptr);
  if (rc) {
    fprintf(stderr, "gpa_decode_step rc=%d: %s\n", rc, last_error.c_str());
    return 3;
  }
  f = fopen(argv[2], "wb");
  for (int64_t i = 0; i < nbuf; ++i) fwrite(buf[i], 1, bytes[i], f);
  fclose(f);
  for (char* b : buf) free(b);
  return 0;
}
