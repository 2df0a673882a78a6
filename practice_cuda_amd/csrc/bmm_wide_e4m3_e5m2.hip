// bmm_wide_e4m3_e5m2.hip - the wide kernel (bmm_wide.h) with an e4m3 A operand and
// an e5m2 B operand.
#include "bmm_wide.h"

namespace pcamd {

int bmm_wide_launch_e4m3_e5m2(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  return bmmw::launch_formats<kE4M3, kE5M2>(a, a_k, b_k, mode, st);
}

}  // namespace pcamd
