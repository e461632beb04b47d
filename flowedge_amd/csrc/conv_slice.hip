// Kernel instances of the sliced fused convolution for Downsample1d (K = 3, stride 2) and
// Upsample1d (ConvTranspose1d K = 4, stride 2) at lengths 2 to 16, and the dispatch over every
// sliced instance (the "same" convolutions live in conv_slice_{s,l}{16,32,64}.hip).  Sliced
// instances exist for the LeRobot U-Net's kernel size 5 and lengths 2 to 16; other shapes run
// unsliced.
#include "conv_kernel.h"

namespace fe::hip::conv {

#define FE_SLICE_SAME(T)                                                                     \
  hipError_t launch_slice_same5_s##T(int lin, int pro, bool res, const Args& a, int batch,  \
                                     hipStream_t s);                                         \
  hipError_t launch_slice_same5_l##T(int lin, int pro, bool res, const Args& a, int batch,  \
                                     hipStream_t s);
FE_SLICE_SAME(16)
FE_SLICE_SAME(32)
FE_SLICE_SAME(64)
#undef FE_SLICE_SAME

bool slice_instance(int mode, int k, int lin, bool res) {
  if (lin != 2 && lin != 4 && lin != 8 && lin != 16) return false;
  if (mode == kConvSame) return k == 5;
  if (res) return false;
  return (mode == kConvDown && k == 3) || (mode == kConvTranspose && k == 4);
}

hipError_t launch_slice(int mode, int k, int lin, int pro, bool res, const Args& a, int batch,
                        hipStream_t s) {
  if (!slice_instance(mode, k, lin, res)) return hipErrorInvalidValue;
  const bool shrt = lin <= 4;
  if (mode == kConvSame) {
    switch (a.tpr) {
      case 16:
        return shrt ? launch_slice_same5_s16(lin, pro, res, a, batch, s)
                    : launch_slice_same5_l16(lin, pro, res, a, batch, s);
      case 32:
        return shrt ? launch_slice_same5_s32(lin, pro, res, a, batch, s)
                    : launch_slice_same5_l32(lin, pro, res, a, batch, s);
      case 64:
        return shrt ? launch_slice_same5_s64(lin, pro, res, a, batch, s)
                    : launch_slice_same5_l64(lin, pro, res, a, batch, s);
      default:
        return hipErrorInvalidValue;
    }
  }
  if (mode == kConvDown) {
    switch (a.tpr) {
      case 16: return slice_lins<kConvDown, 3, 16, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
      case 32: return slice_lins<kConvDown, 3, 32, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
      case 64: return slice_lins<kConvDown, 3, 64, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (a.tpr) {
    case 16: return slice_lins<kConvTranspose, 4, 16, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
    case 32: return slice_lins<kConvTranspose, 4, 32, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
    case 64: return slice_lins<kConvTranspose, 4, 64, 2, 4, 8, 16>(lin, pro, false, a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fe::hip::conv
