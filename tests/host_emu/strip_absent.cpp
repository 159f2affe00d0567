// Host build (test infrastructure): the strip state kernels of
// gdn_state_strip.hip load LDS with global_load_lds from inline assembly and
// exchange lane halves with v_permlane32_swap, which the emulation does not
// model.  Their launchers fail here with a message, so a host test that
// reaches them (bf16 scans of at most 128 keys) fails instead of passing on
// some other path; the scan's other kernels build from their own sources.
#include "gdn_strip.h"
#include "gpa_common.h"

namespace gpa {

int strip_wg_per_stream(int, int) { return 1; }
StripFwdOne strip_fwd_one(const gpa_gdn_problem&, const gpa_gdn_saved&, int, int, int) { return StripFwdOne{}; }
StripBwdOne strip_bwd_one(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int, int, bool, int) {
  return StripBwdOne{};
}

template <int KM>
int launch_state_fwd_strip(const StripFwdPack&, int, bool, int, hipStream_t) {
  return fail(GPA_HIP_EUNSUPPORTED, "host build: the strip state kernels are not emulated");
}
template <int KM>
int launch_state_bwd_strip(const StripBwdPack&, int, bool, bool, bool, int, hipStream_t) {
  return fail(GPA_HIP_EUNSUPPORTED, "host build: the strip state kernels are not emulated");
}
template int launch_state_fwd_strip<64>(const StripFwdPack&, int, bool, int, hipStream_t);
template int launch_state_fwd_strip<128>(const StripFwdPack&, int, bool, int, hipStream_t);
template int launch_state_bwd_strip<64>(const StripBwdPack&, int, bool, bool, bool, int, hipStream_t);
template int launch_state_bwd_strip<128>(const StripBwdPack&, int, bool, bool, bool, int, hipStream_t);

}  // namespace gpa
