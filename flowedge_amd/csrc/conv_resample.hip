// Kernel instances of the fused convolution for Downsample1d (K = 3, stride 2) and Upsample1d
// (ConvTranspose1d K = 4, stride 2).
#include "conv_kernel.h"

namespace fe::hip::conv {

hipError_t launch_resample(int mode, int lin, int pro, const Args& a, int batch, hipStream_t s) {
  if (mode == kConvDown) return by_lin<kConvDown, 3, 4>(lin, pro, false, a, batch, s);
  if (mode == kConvTranspose) return by_lin<kConvTranspose, 4, 4>(lin, pro, false, a, batch, s);
  return hipErrorInvalidValue;
}

}  // namespace fe::hip::conv
