// Kernel instances of the sliced fused convolution: K = 5 "same" convolutions at lengths 2 and 4,
// 32 lanes per row.
#include "conv_kernel.h"

namespace fe::hip::conv {

hipError_t launch_slice_same5_s32(int lin, int pro, bool res, const Args& a, int batch,
                                  hipStream_t s) {
  return slice_lins<kConvSame, 5, 32, 2, 4>(lin, pro, res, a, batch, s);
}

}  // namespace fe::hip::conv
