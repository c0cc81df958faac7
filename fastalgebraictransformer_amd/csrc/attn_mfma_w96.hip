// The MFMA attention kernels for layout width 128, MFMA width 96 (one translation unit per
// width, so that they compile in parallel).

#include "attn_mfma_kernels.h"

namespace kat {
KAT_MFMA_INSTANTIATE(128, 96)
}  // namespace kat
