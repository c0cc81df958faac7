// bf16 / fp16 MFMA rational attention for gfx950: the C-ABI side of the MFMA
// path -- which head dims it takes, the backward's workspace size, the
// 31-bit offset checks, and the dispatch to the layout width and effective
// width a head dim runs in. The kernels and launchers are in
// attn_mfma_kernels.h, instantiated per width in attn_mfma_w*.hip.

#include "attn_mfma_kernels.h"

namespace kat {

KAT_MFMA_WIDTHS(KAT_MFMA_EXTERN)

// head dims that are multiples of 8 up to 256 run in the kernels of the next
// layout width (32, 64, 128 or 256 columns), the columns past D as zeros
bool attn_mfma_supported(int D) { return D >= 8 && D <= 256 && D % 8 == 0; }
bool attn_mfma_fwd_supported(int D) { return attn_mfma_supported(D); }

size_t attn_mfma_workspace(int64_t B, int64_t H, int64_t T, int64_t D, bool causal) {
  return bwd_ws(nullptr, B, H, T, mfma_width(D), causal).bytes;
}

namespace {

// every tensor the kernels read through a buffer resource (q, k, v, and dO and
// O in the backward) must fit 31-bit byte offsets per (b, h) slice and have
// non-overlapping rows
bool offsets_ok(const AttnArgs& a, bool bwd) {
  const int64_t lim = 0x7fffffffLL;
  const int64_t* s2[5] = {&a.sq[2], &a.sk[2], &a.sv[2], &a.sdo[2], &a.so[2]};
  for (int t = 0; t < (bwd ? 5 : 3); ++t)
    if (*s2[t] < a.D || ((int64_t)a.T + std::max(kBM, kFwdBM)) * *s2[t] * 2 > lim) return false;
  return (int64_t)a.T * mfma_width(a.D) * 2 < lim && (int64_t)a.T * 8 < lim;
}

}  // namespace

template <typename T> int attn_fwd_mfma(const AttnArgs& a, hipStream_t st) {
  if ((int64_t)((a.T + kFwdBM - 1) / kFwdBM) * a.B * a.H > 0x7fffffffLL || !offsets_ok(a, false))
    return KAT_EUNSUPPORTED;
  if (!attn_mfma_supported(a.D)) return KAT_EUNSUPPORTED;
  const int W = mfma_width(a.D), E = mfma_eff(a.D);
#define KAT_FWD_CASE(WW, EE) \
  if (W == WW && E == EE) return attn_fwd_w<T, WW, EE>(a, st);
  KAT_MFMA_WIDTHS(KAT_FWD_CASE)
#undef KAT_FWD_CASE
  return KAT_EUNSUPPORTED;
}

template <typename T> int attn_bwd_mfma(const AttnArgs& a, void* ws, hipStream_t st) {
  if ((int64_t)((a.T + 63) / 64) * a.B * a.H > 0x7fffffffLL || !offsets_ok(a, true)) return KAT_EUNSUPPORTED;
  if (!attn_mfma_supported(a.D)) return KAT_EUNSUPPORTED;
  const int W = mfma_width(a.D), E = mfma_eff(a.D);
#define KAT_BWD_CASE(WW, EE) \
  if (W == WW && E == EE) return attn_bwd_w<T, WW, EE>(a, ws, st);
  KAT_MFMA_WIDTHS(KAT_BWD_CASE)
#undef KAT_BWD_CASE
  return KAT_EUNSUPPORTED;
}

template int attn_fwd_mfma<bf16>(const AttnArgs&, hipStream_t);
template int attn_fwd_mfma<f16>(const AttnArgs&, hipStream_t);
template int attn_bwd_mfma<bf16>(const AttnArgs&, void*, hipStream_t);
template int attn_bwd_mfma<f16>(const AttnArgs&, void*, hipStream_t);

}  // namespace kat
