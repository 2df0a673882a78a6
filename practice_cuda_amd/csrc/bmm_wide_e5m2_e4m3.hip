// bmm_wide_e5m2_e4m3.hip - the wide kernel (bmm_wide.h) with an e5m2 A
// operand and an e4m3 B operand: the training recipe's dgrad and wgrad with
// an e5m2 gradient times an e4m3 weight or activation.
#include "bmm_wide.h"

namespace pcamd {

int bmm_wide_launch_e5m2_e4m3(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  return bmmw::launch_formats<kE5M2, kE4M3>(a, a_k, b_k, mode, st);
}

}  // namespace pcamd
