// bmm_wide.hip - the e4m3fn x e4m3fn instantiations of the wide kernel
// (bmm_wide.h) and the dispatch over operand formats.
#include "bmm_wide.h"

namespace pcamd {

int bmm_wide_launch_e5m2(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st);
int bmm_wide_launch_e5m2_e4m3(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st);
int bmm_wide_launch_e4m3_e5m2(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st);

int bmm_wide_launch(const FastArgs& a, int a_fmt, int b_fmt, bool a_k, bool b_k, int mode, hipStream_t st) {
  if (a_fmt == kE4M3 && b_fmt == kE4M3) return bmmw::launch_formats<kE4M3, kE4M3>(a, a_k, b_k, mode, st);
  if (a_fmt == kE5M2 && b_fmt == kE5M2) return bmm_wide_launch_e5m2(a, a_k, b_k, mode, st);
  if (a_fmt == kE5M2 && b_fmt == kE4M3) return bmm_wide_launch_e5m2_e4m3(a, a_k, b_k, mode, st);
  if (a_fmt == kE4M3 && b_fmt == kE5M2) return bmm_wide_launch_e4m3_e5m2(a, a_k, b_k, mode, st);
  return set_error(PCAMD_ERR_INVALID, "bmm_wide: operand formats %d x %d", a_fmt, b_fmt);
}

int bmm_wide_tile() { return bmmw::BM; }

}  // namespace pcamd
