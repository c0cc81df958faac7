// bf16 / fp16 MFMA attention kernels (gfx950).
#include "attn_common.h"
#include "kat_common.h"
#include "kat_internal.h"

namespace kat {

bool attn_mfma_supported(int D) { (void)D; return false; }

template <typename T> int attn_fwd_mfma(const AttnArgs& a, hipStream_t st) {
  (void)a; (void)st;
  return KAT_EUNSUPPORTED;
}
template <typename T> int attn_bwd_mfma(const AttnArgs& a, const float* delta, hipStream_t st) {
  (void)a; (void)delta; (void)st;
  return KAT_EUNSUPPORTED;
}

template int attn_fwd_mfma<bf16>(const AttnArgs&, hipStream_t);
template int attn_fwd_mfma<f16>(const AttnArgs&, hipStream_t);
template int attn_bwd_mfma<bf16>(const AttnArgs&, const float*, hipStream_t);
template int attn_bwd_mfma<f16>(const AttnArgs&, const float*, hipStream_t);

}  // namespace kat
