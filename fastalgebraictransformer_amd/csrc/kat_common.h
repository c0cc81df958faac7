// Shared device helpers for the rational-attention kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kat.h"

namespace kat {

typedef __bf16 bf16;
typedef _Float16 f16;

// ---------------------------------------------------------------------------
// Element types. All arithmetic runs in Acc<T> (fp32, or fp64 for fp64 I/O);
// this matches the reference kernels' `.to(tl.float32)` loads and their store
// in the output tensor's dtype (e.g. fused_ops.py:78,106).
// ---------------------------------------------------------------------------
template <typename T> struct AccT { typedef float type; };
template <> struct AccT<double> { typedef double type; };

template <typename T> __device__ __forceinline__ typename AccT<T>::type to_acc(T x) {
  return (typename AccT<T>::type)x;
}
template <typename T, typename A> __device__ __forceinline__ T from_acc(A x) { return (T)x; }

// 16-byte vector of T (8 x bf16/f16, 4 x f32, 2 x f64) or a single element.
template <typename T, int N> struct __attribute__((aligned(sizeof(T) * N))) VecT {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ void load_acc(const T* __restrict__ p, typename AccT<T>::type (&out)[N]) {
  VecT<T, N> r = *reinterpret_cast<const VecT<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = to_acc(r.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_acc(T* __restrict__ p, const typename AccT<T>::type (&in)[N]) {
  VecT<T, N> r;
#pragma unroll
  for (int i = 0; i < N; ++i) r.v[i] = from_acc<T>(in[i]);
  *reinterpret_cast<VecT<T, N>*>(p) = r;
}

// ---------------------------------------------------------------------------
// Rational sigmoid (fused_ops.py:28-45): sigma(x) = 0.5 * (x / (|x| + 1) + 1).
// The division is kept as an IEEE divide so fp32 results track the
// reference's `x / (abs_x + 1.0)` to the last bit where it matters.
// ---------------------------------------------------------------------------
template <typename A> __device__ __forceinline__ A rsig(A x) {
  return A(0.5) * (x / (fabs(x) + A(1)) + A(1));
}

// a / b in the per-element maps of data of type T. bf16 / fp16 data (results
// rounded to 8 or 11 significand bits) take v_rcp_f32 (1 ulp) and a multiply,
// ~10 instructions fewer than the IEEE divide; fp32 / fp64 data keep the IEEE
// divide (the reference's Triton `/` on fp32 is itself an approximate divide).
template <typename T, typename A> __device__ __forceinline__ A ediv(A a, A b) {
  if constexpr (sizeof(T) == 2 && sizeof(A) == 4)
    return a * __builtin_amdgcn_rcpf(b);
  else
    return a / b;
}
template <typename T, typename A> __device__ __forceinline__ A rsig_t(A x) {
  return A(0.5) * (ediv<T>(x, fabs(x) + A(1)) + A(1));
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) butterfly reduction through cross-lane shuffles.
// ---------------------------------------------------------------------------
template <typename A> __device__ __forceinline__ A wave_sum(A v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace kat
