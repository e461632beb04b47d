// Kernel instances of the fused convolution for K = 5 "same" convolutions.
#include "conv_kernel.h"

namespace fe::hip::conv {

hipError_t launch_same5(int lin, int vec, int pro, bool res, const Args& a, int batch,
                        hipStream_t s) {
  return vec == 4 ? by_lin<kConvSame, 5, 4>(lin, pro, res, a, batch, s)
                  : by_lin<kConvSame, 5, 1>(lin, pro, res, a, batch, s);
}

}  // namespace fe::hip::conv
