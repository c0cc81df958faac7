// The MFMA attention kernels for layout width 256, MFMA width 192 (one translation unit per
// width, so that they compile in parallel).

#include "attn_mfma_kernels.h"

namespace kat {
KAT_MFMA_INSTANTIATE(256, 192)
}  // namespace kat
