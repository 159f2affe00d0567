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
// run it, wg_per_stream = strip_wg_per_stream(V, nq) per stream.
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

// The forms of the strip kernels, by the waves that share a 32-column strip
// (nq): split (2, each with half of the key rows; 64 value columns per
// workgroup), wide (1, every key row; 128 columns) and quarter (4, a quarter of
// the rows each; 32 columns).  A workgroup holds a whole CU (its LDS) and the
// chunk step is bound by each wave's own instruction stream, so fewer rows per
// wave shorten the step while the workgroups fit on the CUs (quarter), and a
// launch that would exceed them runs in the wide form rather than two rounds.
int strip_wg_per_stream(int vdim, int nq);
// Pack entries for one scan group (the buffers of gpa_gdn_saved / gpa_gdn_grads),
// its workgroups starting at wg0.  has_q: the backward has a read gradient.
StripFwdOne strip_fwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, int wg0, int nq);
StripBwdOne strip_bwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          int wg0, bool has_q, int nq);
inline int strip_workgroups(const gpa_gdn_problem& p, int nq) {
  return p.batch * p.heads * strip_wg_per_stream(p.vdim, nq);
}
// Whether a group can run in the wide form (128 keys, V a multiple of 128) or
// the quarter form (128 keys, V a multiple of 64).
inline bool strip_wide_ok(const gpa_gdn_problem& p) { return p.kdim == 128 && p.vdim % 128 == 0; }
inline bool strip_quarter_ok(const gpa_gdn_problem& p) { return p.kdim == 128 && p.vdim % 64 == 0; }
// All groups of a pack share the key-width class KM (K <= KM, K % 16 == 0);
// `fast` when every group has K == KM and V % 64 == 0; nq selects the form
// (1 and 4: KM = 128 and fast; 1: every group strip_wide_ok and, backward,
// no state injections).
template <int KM>
int launch_state_fwd_strip(const StripFwdPack& pk, int total_wg, bool fast, int nq, hipStream_t st);
template <int KM>
int launch_state_bwd_strip(const StripBwdPack& pk, int total_wg, bool fast, bool has_q, bool has_inj, int nq,
                           hipStream_t st);

}  // namespace gpa
