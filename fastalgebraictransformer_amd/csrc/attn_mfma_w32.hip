// The MFMA attention kernels for layout width 32, MFMA width 32, layout width 64, MFMA width 64 (one translation unit per
// width, so that they compile in parallel).

#include "attn_mfma_kernels.h"

namespace kat {
KAT_MFMA_INSTANTIATE(32, 32)
KAT_MFMA_INSTANTIATE(64, 64)
}  // namespace kat
