// Packs of scan groups for the strip state-recurrence kernels (gdn_state_strip.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gpa_hip.h"

namespace gpa {

constexpr int GPA_STRIP_MAXP = 12;  // scan groups per launch

// One scan group of a forward pack: widths, geometry, the initial state
// (key-major, may be null) and the buffers of include/gpa_hip.h's
// gpa_gdn_saved that the recurrence reads (wrow, kcol, u, gam) and writes
// (delta, states, final).  Workgroups wg0 .. wg0 + streams * wg_per_stream - 1
// run it, wg_per_stream = strip_wg_per_stream(V, wide) per stream.
struct StripFwdOne {
  int K, V, heads, nch, wg0, wg_per_stream;
  const float* s0;
  int64_t s0_sb, s0_sh;
  const __bf16* wrow;
  const __bf16* kcol;
  const float* u;
  const float* gam;
  float* delta;
  float* states;
  float* final_state;
};
struct StripFwdPack {
  int n;
  StripFwdOne p[GPA_STRIP_MAXP];
};

// One scan group of a backward pack: dfinal / dstates may be null, dd0 and o
// are read when the group has a read gradient (qcol then holds Qn^T).
struct StripBwdOne {
  int K, V, heads, nch, wg0, wg_per_stream;
  const float* dfinal;
  const float* dstates;
  const float* dd0;
  const float* o;
  float* ddelta;
  float* dhend;
  float* ds0;
  const __bf16* krow;
  const __bf16* wcol;
  const __bf16* qcol;
  const float* gam;
};
struct StripBwdPack {
  int n;
  StripBwdOne p[GPA_STRIP_MAXP];
};

// Workgroups per stream: the split form covers 64 value columns per workgroup
// (two waves per 32-column strip, each with half of the key rows), the wide
// form 128 (one wave per strip with every key row).  A workgroup holds a
// whole CU (its LDS), so a launch of more workgroups than the device has CUs
// runs its chains in two rounds; the wide form halves the workgroups for
// such launches at the cost of a longer chunk step per wave.
int strip_wg_per_stream(int vdim, bool wide);
// Pack entries for one scan group (the buffers of gpa_gdn_saved / gpa_gdn_grads),
// its workgroups starting at wg0.  has_q: the backward has a read gradient.
StripFwdOne strip_fwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, int wg0, bool wide);
StripBwdOne strip_bwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          int wg0, bool has_q, bool wide);
inline int strip_workgroups(const gpa_gdn_problem& p, bool wide) {
  return p.batch * p.heads * strip_wg_per_stream(p.vdim, wide);
}
// Whether a group can run in the wide form: 128 keys, V a multiple of 128.
inline bool strip_wide_ok(const gpa_gdn_problem& p) { return p.kdim == 128 && p.vdim % 128 == 0; }
// All groups of a pack share the key-width class KM (K <= KM, K % 16 == 0);
// `fast` when every group has K == KM and V % 64 == 0; `wide` (KM = 128, every
// group strip_wide_ok, the backward without state injections) selects the
// wide form.
template <int KM>
int launch_state_fwd_strip(const StripFwdPack& pk, int total_wg, bool fast, bool wide, hipStream_t st);
template <int KM>
int launch_state_bwd_strip(const StripBwdPack& pk, int total_wg, bool fast, bool has_q, bool has_inj, bool wide,
                           hipStream_t st);

}  // namespace gpa
