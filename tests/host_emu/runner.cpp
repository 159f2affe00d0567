// Runs one entry point of the host build of the library on a dump (test
// infrastructure).  Dump: the entry point's index; its struct arguments as
// blobs; the buffers (each allocated here with its exact size, so
// AddressSanitizer bounds every access); the pointer fields of the blobs and
// the raw pointer arguments as (buffer, byte offset).  Writes every buffer back.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "gpa_hip.h"

thread_local EmuIdx threadIdx, blockIdx, blockDim, gridDim;
std::barrier<>* emu_block_barrier;
std::vector<std::unique_ptr<std::barrier<>>> emu_wave_barrier;
float emu_xchg[16][64];
float emu_ma[16][64][8], emu_mb[16][64][8];
char* emu_dynamic_lds;
thread_local const void* emu_kernarg;
static std::string last_error;
int fail(int code, const char* message) {
  last_error = message;
  return code;
}
int check_launch(const char*) { return 0; }
void mark(gpa_timing*, hipStream_t) {}  // the host tests pass no timing record

static int64_t get(FILE* f) {
  int64_t x = 0;
  if (fread(&x, 8, 1, f) != 1) exit(4);
  return x;
}

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 2;
  const int64_t entry = get(f);
  std::vector<std::vector<char>> blobs(get(f));
  for (auto& b : blobs) {
    b.resize(get(f));
    if (fread(b.data(), 1, b.size(), f) != b.size()) return 4;
  }
  const int64_t nbuf = get(f);
  std::vector<char*> buf(nbuf);
  std::vector<int64_t> bytes(nbuf);
  for (int64_t i = 0; i < nbuf; ++i) {
    bytes[i] = get(f);
    buf[i] = static_cast<char*>(malloc(bytes[i]));
    if (fread(buf[i], 1, bytes[i], f) != (size_t)bytes[i]) return 4;
  }
  for (auto& b : blobs) {
    const int64_t nptr = get(f);
    for (int64_t i = 0; i < nptr; ++i) {
      const int64_t off = get(f), id = get(f), boff = get(f);
      char* p = buf[id] + boff;
      memcpy(b.data() + off, &p, 8);
    }
  }
  std::vector<void*> raw(get(f));
  for (auto& r : raw) {
    const int64_t id = get(f), boff = get(f);
    r = id < 0 ? nullptr : buf[id] + boff;
  }
  fclose(f);
  int rc = -1;
  int64_t value = 0;  // the result of an entry point that returns a value
  switch (entry) {
    case 0:
      rc = gpa_decode_step(reinterpret_cast<gpa_decode_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 1:
      rc = gpa_route_forward(reinterpret_cast<gpa_route_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 2:
      rc = gpa_route_backward(reinterpret_cast<gpa_route_problem*>(blobs.at(0).data()),
                              reinterpret_cast<gpa_route_grads*>(blobs.at(1).data()), nullptr);
      break;
    case 3:
      rc = gpa_route_weight_grads(reinterpret_cast<gpa_route_problem*>(blobs.at(0).data()),
                                  reinterpret_cast<gpa_route_grads*>(blobs.at(1).data()),
                                  static_cast<float*>(raw.at(0)), static_cast<float*>(raw.at(1)),
                                  static_cast<float*>(raw.at(2)), static_cast<float*>(raw.at(3)), nullptr);
      break;
    case 4:
      rc = gpa_level_forward(reinterpret_cast<gpa_level_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 5:
      rc = gpa_level_backward(reinterpret_cast<gpa_level_problem*>(blobs.at(0).data()),
                              reinterpret_cast<gpa_level_grads*>(blobs.at(1).data()), nullptr);
      break;
    case 6:
      rc = gpa_route_forward_many(reinterpret_cast<gpa_route_problem*>(blobs.at(0).data()),
                                  (int32_t)(blobs.at(0).size() / sizeof(gpa_route_problem)), nullptr);
      break;
    case 7:
      rc = gpa_gdn_token_step(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()), static_cast<float*>(raw.at(0)),
                              *reinterpret_cast<gpa_operand*>(blobs.at(1).data()), nullptr);
      break;
    case 8:
      rc = gpa_gdn_token_step_many(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                                   reinterpret_cast<float* const*>(blobs.at(1).data()),
                                   reinterpret_cast<gpa_operand*>(blobs.at(2).data()),
                                   (int32_t)(blobs.at(0).size() / sizeof(gpa_gdn_problem)), nullptr);
      break;
    case 9:
      rc = gpa_level_token_forward(reinterpret_cast<gpa_level_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 10:
      rc = gpa_token_level_forward(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                                   static_cast<float*>(raw.at(0)), *reinterpret_cast<gpa_operand*>(blobs.at(1).data()),
                                   reinterpret_cast<gpa_level_problem*>(blobs.at(2).data()), nullptr);
      break;
    case 11:
      rc = gpa_product_read_forward(reinterpret_cast<gpa_product_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 12:
      rc = gpa_product_read_backward(reinterpret_cast<gpa_product_problem*>(blobs.at(0).data()),
                                     reinterpret_cast<gpa_product_grads*>(blobs.at(1).data()), nullptr);
      break;
    case 13:
      rc = gpa_token_slot_step(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                               reinterpret_cast<gpa_token_slot*>(blobs.at(1).data()), static_cast<float*>(raw.at(0)),
                               *reinterpret_cast<gpa_operand*>(blobs.at(2).data()),
                               blobs.size() > 3 ? reinterpret_cast<gpa_level_problem*>(blobs.at(3).data()) : nullptr,
                               nullptr);
      break;
    case 14:
      rc = gpa_slot_gates_act_forward(reinterpret_cast<gpa_slot_problem*>(blobs.at(0).data()),
                                      reinterpret_cast<gpa_gate_problem*>(blobs.at(1).data()), nullptr);
      break;
    case 15:
      rc = gpa_moment_scan_many(reinterpret_cast<gpa_moment_problem*>(blobs.at(0).data()),
                                (int32_t)(blobs.at(0).size() / sizeof(gpa_moment_problem)), nullptr);
      break;
    case 16:
      rc = gpa_quad_features_forward(reinterpret_cast<gpa_quad_problem*>(blobs.at(0).data()), nullptr);
      break;
    case 17:
      rc = gpa_quad_features_backward(reinterpret_cast<gpa_quad_problem*>(blobs.at(0).data()),
                                      reinterpret_cast<gpa_quad_grads*>(blobs.at(1).data()), nullptr);
      break;
    case 18:
      rc = gpa_gdn_forward(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                           reinterpret_cast<gpa_gdn_saved*>(blobs.at(1).data()),
                           *reinterpret_cast<gpa_operand*>(blobs.at(2).data()), nullptr, nullptr);
      break;
    case 19:
      rc = gpa_gdn_backward(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                            reinterpret_cast<gpa_gdn_saved*>(blobs.at(1).data()),
                            reinterpret_cast<gpa_gdn_grads*>(blobs.at(2).data()), nullptr, nullptr);
      break;
    case 20:
      rc = gpa_gdn_forward_many(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                                reinterpret_cast<gpa_gdn_saved*>(blobs.at(1).data()),
                                reinterpret_cast<gpa_operand*>(blobs.at(2).data()),
                                (int32_t)(blobs.at(0).size() / sizeof(gpa_gdn_problem)), nullptr, nullptr);
      break;
    case 21:
      rc = gpa_gdn_backward_many(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()),
                                 reinterpret_cast<gpa_gdn_saved*>(blobs.at(1).data()),
                                 reinterpret_cast<gpa_gdn_grads*>(blobs.at(2).data()),
                                 (int32_t)(blobs.at(0).size() / sizeof(gpa_gdn_problem)), nullptr, nullptr);
      break;
    case 22: {
      const int32_t* a = reinterpret_cast<const int32_t*>(blobs.at(0).data());
      value = gpa_gdn_nchunks(a[0], a[1], a[2]);
      rc = 0;
      break;
    }
    case 23:
      value = gpa_gdn_path(reinterpret_cast<gpa_gdn_problem*>(blobs.at(0).data()));
      rc = 0;
      break;
  }
  if (rc) {
    fprintf(stderr, "entry %ld rc=%d: %s\n", (long)entry, rc, last_error.c_str());
    return 3;
  }
  f = fopen(argv[2], "wb");
  for (int64_t i = 0; i < nbuf; ++i) fwrite(buf[i], 1, bytes[i], f);
  fclose(f);
  for (char* b : buf) free(b);
  printf("%lld\n", (long long)value);
  return 0;
}
