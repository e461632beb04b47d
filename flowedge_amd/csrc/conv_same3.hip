// Kernel instances of the fused convolution for K = 3 "same" convolutions.
#include "conv_kernel.h"

namespace fe::hip::conv {

hipError_t launch_same3(int lin, int vec, int pro, bool res, const Args& a, int batch,
                        hipStream_t s) {
  return vec == 4 ? by_lin<kConvSame, 3, 4>(lin, pro, res, a, batch, s)
                  : by_lin<kConvSame, 3, 1>(lin, pro, res, a, batch, s);
}

}  // namespace fe::hip::conv
