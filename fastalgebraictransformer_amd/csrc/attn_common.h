// Argument block shared by the attention kernels and their launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kat_common.h"

namespace kat {

// Layout [B, H, T, D]: element (b, h, t, d) of tensor X sits at
// X + b*sX[0] + h*sX[1] + t*sX[2] + d (unit d-stride). L: [B, H, T] fp32.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;           // forward output / backward input O
  const void* dout;  // backward only
  void* dq;
  void* dk;
  void* dv;
  float* L;
  const float* slopes;
  int B, H, T, D;
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sdq[3], sdk[3], sdv[3], sl[3];
  float scale, eps;
  // key padding mask: key j of batch b is attended iff km[b * skm + j] != 0
  // (km == nullptr: every key); causal == 0: every key visible, ALiBi on |i - j|
  const uint8_t* km;
  int64_t skm;
  int causal;
};

// key j of batch b passes the padding mask (j < T assumed)
__device__ __forceinline__ bool key_ok(const AttnArgs& a, int b, int j) {
  return a.km == nullptr || a.km[(int64_t)b * a.skm + j] != 0;
}

// Tiled kernels (any D <= 1024; fp32 arithmetic, fp64 for double tensors).
template <typename T> int attn_fwd_generic(const AttnArgs& a, hipStream_t st);
// Delta_i = <dO_i, O_i> and cinv_i = 1 / (16 (L_i + eps)), both [B*H*T] in the
// accumulation type (fp32, fp64 for double tensors).
template <typename T>
int attn_delta(const AttnArgs& a, typename AccT<T>::type* delta, typename AccT<T>::type* cinv, hipStream_t st);
template <typename T>
int attn_bwd_generic(const AttnArgs& a, const typename AccT<T>::type* delta, hipStream_t st);

// bf16 / fp16 MFMA kernels; return KAT_EUNSUPPORTED when the shape is not covered.
// The backward runs its own prep pass; ws holds attn_mfma_workspace() bytes for
// the call's mode: per-row stats (per 64-row tile: 4 cinv, then -4 cinv Delta),
// an fp16 copy of Q ([B*H][T][W], W the layout width 32, 64, 128 or 256 the
// head dim runs in, columns past D zero),
// per-tile exponents and dS-bound parts, per-32-key K exponents, the fp16 dS
// tiles of a group of heads or of one band of a head's keys (at most 4 GiB of
// them, or one band of 512 keys), and for banded calls one head's fp32 dQ
// partial sums.
template <typename T> int attn_fwd_mfma(const AttnArgs& a, hipStream_t st);
template <typename T> int attn_bwd_mfma(const AttnArgs& a, void* ws, hipStream_t st);
bool attn_mfma_supported(int D);      // head dims of the MFMA kernels: multiples of 8 up to 256
bool attn_mfma_fwd_supported(int D);  // the same set, for the forward's dispatch
size_t attn_mfma_workspace(int64_t B, int64_t H, int64_t T, int64_t D, bool causal);

// fp32 forward and backward on the fp32 matrix instruction (head dims:
// multiples of 4 up to 256); KAT_EUNSUPPORTED when the shape is not covered.
// The backward takes Delta and cinv from attn_delta<float>.
bool attn_f32_mfma_supported(int D);
int attn_fwd_mfma_f32(const AttnArgs& a, hipStream_t st);
int attn_bwd_mfma_f32(const AttnArgs& a, const float* delta, const float* cinv, hipStream_t st);

}  // namespace kat
