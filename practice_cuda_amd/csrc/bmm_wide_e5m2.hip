// bmm_wide_e5m2.hip - the e5m2 x e5m2 instantiations of the wide kernel
// (bmm_wide.h).
#include "bmm_wide.h"

namespace pcamd {

int bmm_wide_launch_e5m2(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  return bmmw::launch_formats<kE5M2, kE5M2>(a, a_k, b_k, mode, st);
}

}  // namespace pcamd
