// C ABI of the rational-attention kernels: argument checks and kernel choice.
//
// Kernel choice: bf16 / fp16 tensors with a head dim the MFMA kernels cover
// (and 16-byte aligned rows) go to the MFMA kernels, and so do fp32 tensors
// (the fp32 matrix instruction; head dims that are multiples of 4 up to 256);
// everything else (fp64, other head dims up to 1024, unaligned views) to the
// tiled kernels (fp32 arithmetic; fp64 for fp64 tensors).
// KAT_ATTN_IMPL in the environment overrides the choice: "tiled" forces the
// tiled kernels, "mfma" makes a bf16 / fp16 / fp32 call that cannot take the
// MFMA kernels fail with KAT_EUNSUPPORTED instead of falling back (both used
// by the tests to pin which kernels they exercise).

#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "attn_common.h"
#include "kat_common.h"
#include "kat_internal.h"

using namespace kat;

namespace {

bool force_tiled() {
  const char* e = getenv("KAT_ATTN_IMPL");
  return e && strcmp(e, "tiled") == 0;
}
bool require_mfma() {
  const char* e = getenv("KAT_ATTN_IMPL");
  return e && strcmp(e, "mfma") == 0;
}

int fill_args(const char* nm, AttnArgs& a, int64_t B, int64_t H, int64_t T, int64_t D,
              const int64_t* strides, int n_tensors, const int64_t* l_strides) {
  if (B < 0 || H < 0 || T < 0 || D < 0) return fail(KAT_EINVAL, "%s: negative size", nm);
  if (B * H > 0x7fffffffLL || T > 0x7fffffffLL)
    return fail(KAT_EUNSUPPORTED, "%s: B*H or T too large", nm);
  if (D > 1024) return fail(KAT_EUNSUPPORTED, "%s: head dim %lld > 1024", nm, (long long)D);
  if (!strides || !l_strides) return fail(KAT_EINVAL, "%s: null stride array", nm);
  a.B = (int)B;
  a.H = (int)H;
  a.T = (int)T;
  a.D = (int)D;
  int64_t* dst[8] = {a.sq, a.sk, a.sv, a.so, a.sdo, a.sdq, a.sdk, a.sdv};
  const int order_fwd[4] = {0, 1, 2, 3};  // q, k, v, out
  for (int t = 0; t < 8; ++t)
    for (int j = 0; j < 3; ++j) dst[t][j] = 0;
  for (int t = 0; t < n_tensors; ++t) {
    const int slot = n_tensors == 4 ? order_fwd[t] : t;
    for (int j = 0; j < 3; ++j) dst[slot][j] = strides[3 * t + j];
  }
  for (int j = 0; j < 3; ++j) a.sl[j] = l_strides[j];
  return KAT_OK;
}

template <typename T> bool rows16(const void* p, const int64_t* s) {
  return aligned16(p) && (s[0] * (int64_t)sizeof(T)) % 16 == 0 &&
         (s[1] * (int64_t)sizeof(T)) % 16 == 0 && (s[2] * (int64_t)sizeof(T)) % 16 == 0;
}

// workspace of the tiled path: Delta [B*H*T], then cinv [B*H*T] (each 256-byte
// aligned; fp32, fp64 for fp64 tensors); the MFMA path lays out its own
// (attn_mfma_workspace), sized for the call's mode (causal or not). One buffer
// of the larger size serves whichever path a call takes.
size_t stat_bytes(int64_t B, int64_t H, int64_t T, int dtype) {
  const size_t e = dtype == KAT_F64 ? sizeof(double) : sizeof(float);
  return (((size_t)(B * H * T) * e) + 255) & ~(size_t)255;
}
size_t delta_bytes(int64_t B, int64_t H, int64_t T, int dtype) { return 2 * stat_bytes(B, H, T, dtype); }
size_t bwd_workspace(int64_t B, int64_t H, int64_t T, int64_t D, int dtype, bool causal) {
  size_t n = delta_bytes(B, H, T, dtype);
  if ((dtype == KAT_BF16 || dtype == KAT_F16) && attn_mfma_supported((int)D))
    n = std::max(n, attn_mfma_workspace(B, H, T, D, causal));
  return n;
}

}  // namespace

template <typename T> static int attn_fwd_t(const AttnArgs& a, hipStream_t st) {
  if (!force_tiled() && attn_mfma_fwd_supported(a.D) && rows16<T>(a.q, a.sq) &&
      rows16<T>(a.k, a.sk) && rows16<T>(a.v, a.sv) && rows16<T>(a.o, a.so)) {
    const int rc = attn_fwd_mfma<T>(a, st);
    if (rc != KAT_EUNSUPPORTED) return rc;
  }
  if (require_mfma()) return fail(KAT_EUNSUPPORTED, "kat_attn_fwd: shape / layout not covered by the MFMA kernels");
  return attn_fwd_generic<T>(a, st);
}

static int attn_fwd_f32(const AttnArgs& a, hipStream_t st) {
  if (!force_tiled() && attn_f32_mfma_supported(a.D) && rows16<float>(a.q, a.sq) &&
      rows16<float>(a.k, a.sk) && rows16<float>(a.v, a.sv) && rows16<float>(a.o, a.so)) {
    const int rc = attn_fwd_mfma_f32(a, st);
    if (rc != KAT_EUNSUPPORTED) return rc;
  }
  if (require_mfma()) return fail(KAT_EUNSUPPORTED, "kat_attn_fwd: shape / layout not covered by the fp32 MFMA kernel");
  return attn_fwd_generic<float>(a, st);
}

// Delta and cinv (accumulation type) at the start of the workspace, then the
// tiled backward kernels
template <typename T>
static int attn_bwd_tiled(const AttnArgs& a, void* ws, hipStream_t st) {
  typedef typename AccT<T>::type A;
  const int dt = sizeof(A) == 8 ? KAT_F64 : KAT_F32;
  A* delta = reinterpret_cast<A*>(ws);
  A* cinv = reinterpret_cast<A*>(reinterpret_cast<char*>(ws) + stat_bytes(a.B, a.H, a.T, dt));
  if (int rc = attn_delta<T>(a, delta, cinv, st)) return rc;
  return attn_bwd_generic<T>(a, delta, st);
}

static int attn_bwd_f32(const AttnArgs& a, void* ws, hipStream_t st) {
  if (!force_tiled() && attn_f32_mfma_supported(a.D) && rows16<float>(a.q, a.sq) &&
      rows16<float>(a.k, a.sk) && rows16<float>(a.v, a.sv) && rows16<float>(a.dout, a.sdo) &&
      rows16<float>(a.dq, a.sdq) && rows16<float>(a.dk, a.sdk) && rows16<float>(a.dv, a.sdv)) {
    float* delta = reinterpret_cast<float*>(ws);
    float* cinv = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + stat_bytes(a.B, a.H, a.T, KAT_F32));
    if (int rc = attn_delta<float>(a, delta, cinv, st)) return rc;
    const int rc = attn_bwd_mfma_f32(a, delta, cinv, st);
    if (rc != KAT_EUNSUPPORTED) return rc;
  }
  if (require_mfma()) return fail(KAT_EUNSUPPORTED, "kat_attn_bwd: shape / layout not covered by the fp32 MFMA kernels");
  return attn_bwd_tiled<float>(a, ws, st);
}

template <typename T>
static int attn_bwd_t(const AttnArgs& a, void* ws, hipStream_t st) {
  if (!force_tiled() && attn_mfma_supported(a.D) && rows16<T>(a.q, a.sq) &&
      rows16<T>(a.k, a.sk) && rows16<T>(a.v, a.sv) && rows16<T>(a.o, a.so) &&
      rows16<T>(a.dout, a.sdo) && rows16<T>(a.dq, a.sdq) && rows16<T>(a.dk, a.sdk) &&
      rows16<T>(a.dv, a.sdv)) {
    const int rc = attn_bwd_mfma<T>(a, ws, st);
    if (rc != KAT_EUNSUPPORTED) return rc;
  }
  if (require_mfma()) return fail(KAT_EUNSUPPORTED, "kat_attn_bwd: shape / layout not covered by the MFMA kernels");
  return attn_bwd_tiled<T>(a, ws, st);
}

static int attn_fwd_impl(const char* nm, const void* q, const void* k, const void* v, void* out,
                         float* L, const float* slopes, const uint8_t* key_mask,
                         int64_t mask_stride_b, int64_t B, int64_t H, int64_t T, int64_t D,
                         const int64_t* strides, const int64_t* l_strides, float scale, float eps,
                         int causal, int dtype, void* stream) {
  AttnArgs a = {};
  if (int rc = fill_args(nm, a, B, H, T, D, strides, 4, l_strides)) return rc;
  if (B * H * T == 0 || D == 0) return KAT_OK;
  if (!q || !k || !v || !out || !L || !slopes) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (key_mask && mask_stride_b < T && B > 1)
    return fail(KAT_EINVAL, "%s: key-mask batch stride %lld < T %lld", nm, (long long)mask_stride_b,
                (long long)T);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.L = L;
  a.slopes = slopes;
  a.scale = scale;
  a.eps = eps;
  a.km = key_mask;
  a.skm = mask_stride_b;
  a.causal = causal ? 1 : 0;
  const hipStream_t st = as_stream(stream);
  switch (dtype) {
    case KAT_F32: return attn_fwd_f32(a, st);
    case KAT_F64: return attn_fwd_generic<double>(a, st);
    case KAT_BF16: return attn_fwd_t<bf16>(a, st);
    case KAT_F16: return attn_fwd_t<f16>(a, st);
    default: return fail(KAT_EUNSUPPORTED, "%s: unsupported dtype %d", nm, dtype);
  }
}

extern "C" int kat_attn_fwd(const void* q, const void* k, const void* v, void* out, float* L,
                            const float* slopes, int64_t B, int64_t H, int64_t T, int64_t D,
                            const int64_t* strides, const int64_t* l_strides, float scale,
                            float eps, int causal, int dtype, void* stream) {
  (void)causal;  // always causal, as the reference (forward.py:110)
  return attn_fwd_impl("kat_attn_fwd", q, k, v, out, L, slopes, nullptr, 0, B, H, T, D, strides,
                       l_strides, scale, eps, 1, dtype, stream);
}

extern "C" int kat_attn_fwd_masked(const void* q, const void* k, const void* v, void* out,
                                   float* L, const float* slopes, const uint8_t* key_mask,
                                   int64_t mask_stride_b, int64_t B, int64_t H, int64_t T,
                                   int64_t D, const int64_t* strides, const int64_t* l_strides,
                                   float scale, float eps, int causal, int dtype, void* stream) {
  return attn_fwd_impl("kat_attn_fwd_masked", q, k, v, out, L, slopes, key_mask, mask_stride_b, B,
                       H, T, D, strides, l_strides, scale, eps, causal, dtype, stream);
}

extern "C" size_t kat_attn_bwd_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D,
                                              int dtype) {
  if (B <= 0 || H <= 0 || T <= 0 || D < 0) return 0;
  return bwd_workspace(B, H, T, D, dtype, true);
}

extern "C" size_t kat_attn_bwd_masked_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D,
                                                     int dtype, int causal) {
  if (B <= 0 || H <= 0 || T <= 0 || D < 0) return 0;
  return bwd_workspace(B, H, T, D, dtype, causal != 0);
}

static int attn_bwd_impl(const char* nm, const void* q, const void* k, const void* v,
                         const void* out, const float* L, const void* dout, void* dq, void* dk,
                         void* dv, const float* slopes, const uint8_t* key_mask,
                         int64_t mask_stride_b, void* workspace, size_t workspace_bytes,
                         int64_t B, int64_t H, int64_t T, int64_t D, const int64_t* strides,
                         const int64_t* l_strides, float scale, float eps, int causal, int dtype,
                         void* stream) {
  AttnArgs a = {};
  if (int rc = fill_args(nm, a, B, H, T, D, strides, 8, l_strides)) return rc;
  if (B * H * T == 0 || D == 0) return KAT_OK;
  if (!q || !k || !v || !out || !L || !dout || !dq || !dk || !dv || !slopes)
    return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (key_mask && mask_stride_b < T && B > 1)
    return fail(KAT_EINVAL, "%s: key-mask batch stride %lld < T %lld", nm, (long long)mask_stride_b,
                (long long)T);
  const size_t need = bwd_workspace(B, H, T, D, dtype, causal != 0);
  if (!workspace || workspace_bytes < need)
    return fail(KAT_EINVAL, "%s: workspace %zu bytes < required %zu", nm, workspace_bytes, need);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = const_cast<void*>(out);
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.L = const_cast<float*>(L);
  a.slopes = slopes;
  a.scale = scale;
  a.eps = eps;
  a.km = key_mask;
  a.skm = mask_stride_b;
  a.causal = causal ? 1 : 0;
  const hipStream_t st = as_stream(stream);
  switch (dtype) {
    case KAT_F32: return attn_bwd_f32(a, workspace, st);
    case KAT_F64: return attn_bwd_tiled<double>(a, workspace, st);
    case KAT_BF16: return attn_bwd_t<bf16>(a, workspace, st);
    case KAT_F16: return attn_bwd_t<f16>(a, workspace, st);
    default: return fail(KAT_EUNSUPPORTED, "%s: unsupported dtype %d", nm, dtype);
  }
}

extern "C" int kat_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                            const float* L, const void* dout, void* dq, void* dk, void* dv,
                            const float* slopes, void* workspace, size_t workspace_bytes,
                            int64_t B, int64_t H, int64_t T, int64_t D, const int64_t* strides,
                            const int64_t* l_strides, float scale, float eps, int causal,
                            int dtype, void* stream) {
  (void)causal;  // always causal, as the reference (backward.py:125,222)
  return attn_bwd_impl("kat_attn_bwd", q, k, v, out, L, dout, dq, dk, dv, slopes, nullptr, 0,
                       workspace, workspace_bytes, B, H, T, D, strides, l_strides, scale, eps, 1,
                       dtype, stream);
}

extern "C" int kat_attn_bwd_masked(const void* q, const void* k, const void* v, const void* out,
                                   const float* L, const void* dout, void* dq, void* dk, void* dv,
                                   const float* slopes, const uint8_t* key_mask,
                                   int64_t mask_stride_b, void* workspace, size_t workspace_bytes,
                                   int64_t B, int64_t H, int64_t T, int64_t D,
                                   const int64_t* strides, const int64_t* l_strides, float scale,
                                   float eps, int causal, int dtype, void* stream) {
  return attn_bwd_impl("kat_attn_bwd_masked", q, k, v, out, L, dout, dq, dk, dv, slopes, key_mask,
                       mask_stride_b, workspace, workspace_bytes, B, H, T, D, strides, l_strides,
                       scale, eps, causal, dtype, stream);
}
