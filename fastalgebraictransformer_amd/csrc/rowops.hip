// Bandwidth-bound row operations of the algebraic transformer on gfx950:
// rational softmax, rational SwiGLU and mean-error norm, forward and backward.
//
// Design (MI355X): these ops do a handful of flops per byte, so the only
// roofline that matters is HBM (8 TB/s). Every kernel touches each tensor
// exactly once:
//   * row-resident kernels (softmax, norm): one 64-lane wavefront owns a row,
//     holds it in registers as packed 16-byte vectors, reduces with cross-lane
//     shuffles and writes the result -- one HBM pass where the reference makes
//     two (fused_ops.py:74-106, 319-342, 395-423);
//   * SwiGLU is a flat elementwise stream of 16-byte vectors with row strides,
//     so gate/value can be the two halves of one packed buffer;
//   * the norm backward folds the weight gradient (torch ops at
//     fused_ops.py:593-597 in the reference) into the same pass as per-block
//     column partials, reduced afterwards in a fixed order (deterministic).
// Rows wider than 16 vectors per lane fall back to a multi-pass block-per-row
// kernel that re-reads the row (it stays in L2).

#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "kat_common.h"
#include "kat_internal.h"

namespace kat {

constexpr int kRowWaves = 4;  // waves (rows) per 256-thread block
constexpr int kEwThreads = 256;
constexpr int kEwUnroll = 4;
constexpr int64_t kMaxChunks = 1LL << 30;  // per launch: keeps in-kernel index math 32-bit

template <typename T> struct Raw {
  static constexpr int V = 16 / sizeof(T);
  typedef VecT<T, V> type;
};

template <typename T, int V>
__device__ __forceinline__ VecT<T, V> ld_vec(const T* __restrict__ p) {
  return *reinterpret_cast<const VecT<T, V>*>(p);
}
template <typename T, int V>
__device__ __forceinline__ void st_vec(T* __restrict__ p, const VecT<T, V>& v) {
  *reinterpret_cast<VecT<T, V>*>(p) = v;
}
template <typename T, int V> __device__ __forceinline__ VecT<T, V> zero_vec() {
  VecT<T, V> z;
#pragma unroll
  for (int i = 0; i < V; ++i) z.v[i] = T(0);
  return z;
}

template <typename A> __device__ __forceinline__ A sign_of(A x) {
  // torch.sign semantics (abs backward): sign(0) = 0
  return x > A(0) ? A(1) : (x < A(0) ? A(-1) : A(0));
}

// Block-wide sum for the multi-pass kernels (256 threads).
template <typename A> __device__ A block_sum(A v, A* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  A t = A(0);
#pragma unroll
  for (int i = 0; i < kRowWaves; ++i) t += sh[i];
  return t;
}

// ============================================================================
// rational SwiGLU -- fused_ops.py:196-288
// ============================================================================

template <typename T, int V>
__global__ __launch_bounds__(kEwThreads) void swiglu_fwd_k(
    const T* __restrict__ g, const T* __restrict__ v, T* __restrict__ o, uint32_t n_chunks,
    uint32_t cpr, int64_t ldg, int64_t ldv, int64_t ldo) {
  typedef typename AccT<T>::type A;
  const uint32_t base = blockIdx.x * (kEwThreads * kEwUnroll) + threadIdx.x;
  VecT<T, V> gr[kEwUnroll], vr[kEwUnroll];
  int64_t row[kEwUnroll], col[kEwUnroll];
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    const uint32_t c = base + (uint32_t)u * kEwThreads;
    const bool ok = c < n_chunks;
    const uint32_t cc = ok ? c : 0u;
    const uint32_t r = cc / cpr;
    row[u] = (int64_t)r;
    col[u] = (int64_t)(cc - r * cpr) * V;
    if (ok) {
      gr[u] = ld_vec<T, V>(g + row[u] * ldg + col[u]);
      vr[u] = ld_vec<T, V>(v + row[u] * ldv + col[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    if (base + (uint32_t)u * kEwThreads < n_chunks) {
      VecT<T, V> out;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A gg = to_acc(gr[u].v[i]);
        const A vv = to_acc(vr[u].v[i]);
        out.v[i] = from_acc<T>(gg * rsig(gg) * vv);  // fused_ops.py:224-227
      }
      st_vec<T, V>(o + row[u] * ldo + col[u], out);
    }
  }
}

template <typename T, int V>
__global__ __launch_bounds__(kEwThreads) void swiglu_bwd_k(
    const T* __restrict__ dy, const T* __restrict__ g, const T* __restrict__ v,
    T* __restrict__ dg, T* __restrict__ dv, uint32_t n_chunks, uint32_t cpr, int64_t lddy,
    int64_t ldg, int64_t ldv, int64_t lddg, int64_t lddv) {
  typedef typename AccT<T>::type A;
  const uint32_t base = blockIdx.x * (kEwThreads * kEwUnroll) + threadIdx.x;
  VecT<T, V> yr[kEwUnroll], gr[kEwUnroll], vr[kEwUnroll];
  int64_t row[kEwUnroll], col[kEwUnroll];
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    const uint32_t c = base + (uint32_t)u * kEwThreads;
    const bool ok = c < n_chunks;
    const uint32_t cc = ok ? c : 0u;
    const uint32_t r = cc / cpr;
    row[u] = (int64_t)r;
    col[u] = (int64_t)(cc - r * cpr) * V;
    if (ok) {
      yr[u] = ld_vec<T, V>(dy + row[u] * lddy + col[u]);
      gr[u] = ld_vec<T, V>(g + row[u] * ldg + col[u]);
      vr[u] = ld_vec<T, V>(v + row[u] * ldv + col[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    if (base + (uint32_t)u * kEwThreads < n_chunks) {
      VecT<T, V> og, ov;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A y = to_acc(yr[u].v[i]);
        const A gg = to_acc(gr[u].v[i]);
        const A vv = to_acc(vr[u].v[i]);
        // fused_ops.py:276-285
        const A den = fabs(gg) + A(1);
        const A sig = A(0.5) * (gg / den + A(1));
        const A sd = A(0.5) / (den * den);
        ov.v[i] = from_acc<T>(y * gg * sig);
        og.v[i] = from_acc<T>(y * vv * (sig + gg * sd));
      }
      st_vec<T, V>(dg + row[u] * lddg + col[u], og);
      st_vec<T, V>(dv + row[u] * lddv + col[u], ov);
    }
  }
}

// Scalar fallback for misaligned / odd-width inputs.
template <typename T>
__global__ __launch_bounds__(kEwThreads) void swiglu_fwd_scalar_k(
    const T* __restrict__ g, const T* __restrict__ v, T* __restrict__ o, uint64_t n,
    uint64_t cols, int64_t ldg, int64_t ldv, int64_t ldo) {
  typedef typename AccT<T>::type A;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (uint64_t)gridDim.x * blockDim.x) {
    const int64_t r = (int64_t)(e / cols), c = (int64_t)(e - (uint64_t)r * cols);
    const A gg = to_acc(g[r * ldg + c]), vv = to_acc(v[r * ldv + c]);
    o[r * ldo + c] = from_acc<T>(gg * rsig(gg) * vv);
  }
}

template <typename T>
__global__ __launch_bounds__(kEwThreads) void swiglu_bwd_scalar_k(
    const T* __restrict__ dy, const T* __restrict__ g, const T* __restrict__ v,
    T* __restrict__ dg, T* __restrict__ dv, uint64_t n, uint64_t cols, int64_t lddy, int64_t ldg,
    int64_t ldv, int64_t lddg, int64_t lddv) {
  typedef typename AccT<T>::type A;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (uint64_t)gridDim.x * blockDim.x) {
    const int64_t r = (int64_t)(e / cols), c = (int64_t)(e - (uint64_t)r * cols);
    const A y = to_acc(dy[r * lddy + c]), gg = to_acc(g[r * ldg + c]), vv = to_acc(v[r * ldv + c]);
    const A den = fabs(gg) + A(1);
    const A sig = A(0.5) * (gg / den + A(1));
    const A sd = A(0.5) / (den * den);
    dv[r * lddv + c] = from_acc<T>(y * gg * sig);
    dg[r * lddg + c] = from_acc<T>(y * vv * (sig + gg * sd));
  }
}

// ============================================================================
// rational softmax -- fused_ops.py:52-189
// ============================================================================

template <typename T, int NCH>
__global__ __launch_bounds__(256) void rsoftmax_fwd_k(const T* __restrict__ x, T* __restrict__ p,
                                                      int64_t n_rows, int n_cols, int64_t ldx,
                                                      int64_t ldp, float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const T* xr = x + row * ldx;
  VecT<T, V> raw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    raw[c] = col < n_cols ? ld_vec<T, V>(xr + col) : zero_vec<T, V>();
  }
  A f[NCH][V];
  A sum = A(0);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool in = (c * 64 + lane) * V < n_cols;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const A s = rsig(to_acc(raw[c].v[i]));  // fused_ops.py:81-86
      const A s2 = s * s;
      f[c][i] = s2 * s2;
      sum += in ? f[c][i] : A(0);
    }
  }
  sum = wave_sum(sum);
  const A inv = A(1) / (sum + A(eps));  // fused_ops.py:90
  T* pr = p + row * ldp;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    if (col < n_cols) {
      VecT<T, V> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = from_acc<T>(f[c][i] * inv);  // fused_ops.py:104
      st_vec<T, V>(pr + col, o);
    }
  }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void rsoftmax_bwd_k(const T* __restrict__ dy,
                                                      const T* __restrict__ x,
                                                      const T* __restrict__ p, T* __restrict__ dx,
                                                      int64_t n_rows, int n_cols, int64_t lddy,
                                                      int64_t ldx, int64_t ldp, int64_t lddx,
                                                      float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  VecT<T, V> ry[NCH], rp[NCH], rx[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    const bool in = col < n_cols;
    ry[c] = in ? ld_vec<T, V>(dy + row * lddy + col) : zero_vec<T, V>();
    rp[c] = in ? ld_vec<T, V>(p + row * ldp + col) : zero_vec<T, V>();
    rx[c] = in ? ld_vec<T, V>(x + row * ldx + col) : zero_vec<T, V>();
  }
  A dot = A(0);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) dot += to_acc(ry[c].v[i]) * to_acc(rp[c].v[i]);  // :167
  dot = wave_sum(dot);
  const A e = A(eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    if (col < n_cols) {
      VecT<T, V> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A xx = to_acc(rx[c].v[i]);
        const A den = fabs(xx) + A(1);  // fused_ops.py:179-187
        const A sig = A(0.5) * (xx / den + A(1));
        const A g = A(2) / (den * den * (sig + e));
        o.v[i] = from_acc<T>(to_acc(rp[c].v[i]) * g * (to_acc(ry[c].v[i]) - dot));
      }
      st_vec<T, V>(dx + row * lddx + col, o);
    }
  }
}

// Multi-pass block-per-row fallbacks (wide rows, misaligned or odd widths).
template <typename T>
__global__ __launch_bounds__(256) void rsoftmax_fwd_mp_k(const T* __restrict__ x,
                                                         T* __restrict__ p, int64_t n_rows,
                                                         int n_cols, int64_t ldx, int64_t ldp,
                                                         float eps) {
  typedef typename AccT<T>::type A;
  __shared__ A sh[kRowWaves];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  A sum = A(0);
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
    const A s = rsig(to_acc(xr[c]));
    const A s2 = s * s;
    sum += s2 * s2;
  }
  sum = block_sum(sum, sh);
  const A inv = A(1) / (sum + A(eps));
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
    const A s = rsig(to_acc(xr[c]));
    const A s2 = s * s;
    p[row * ldp + c] = from_acc<T>(s2 * s2 * inv);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rsoftmax_bwd_mp_k(const T* __restrict__ dy,
                                                         const T* __restrict__ x,
                                                         const T* __restrict__ p,
                                                         T* __restrict__ dx, int64_t n_rows,
                                                         int n_cols, int64_t lddy, int64_t ldx,
                                                         int64_t ldp, int64_t lddx, float eps) {
  typedef typename AccT<T>::type A;
  __shared__ A sh[kRowWaves];
  const int64_t row = blockIdx.x;
  A dot = A(0);
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x)
    dot += to_acc(dy[row * lddy + c]) * to_acc(p[row * ldp + c]);
  dot = block_sum(dot, sh);
  const A e = A(eps);
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
    const A xx = to_acc(x[row * ldx + c]);
    const A den = fabs(xx) + A(1);
    const A sig = A(0.5) * (xx / den + A(1));
    const A g = A(2) / (den * den * (sig + e));
    dx[row * lddx + c] =
        from_acc<T>(to_acc(p[row * ldp + c]) * g * (to_acc(dy[row * lddy + c]) - dot));
  }
}

// ============================================================================
// mean-error norm -- fused_ops.py:295-423 (+ dgamma, fused_ops.py:593-597)
// ============================================================================

template <typename T, typename W, int NCH>
__global__ __launch_bounds__(256) void men_fwd_k(const T* __restrict__ x, const W* __restrict__ w,
                                                 T* __restrict__ y, float* __restrict__ mu,
                                                 int64_t n_rows, int n_cols, int64_t ldx,
                                                 int64_t ldy, float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  VecT<T, V> rx[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    rx[c] = col < n_cols ? ld_vec<T, V>(x + row * ldx + col) : zero_vec<T, V>();
  }
  A s = A(0);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) s += fabs(to_acc(rx[c].v[i]));  // fused_ops.py:324
  s = wave_sum(s);
  const A mean = s / A(n_cols);                  // fused_ops.py:326
  const A inv = A(1) / (mean + A(eps));          // fused_ops.py:327
  if (lane == 0) mu[row] = (float)mean;          // fused_ops.py:330 (no eps)
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
    if (col < n_cols) {
      VecT<T, V> o;
#pragma unroll
      for (int i = 0; i < V; ++i)
        o.v[i] = from_acc<T>(to_acc(rx[c].v[i]) * inv * (A)w[col + i]);  // :340
      st_vec<T, V>(y + row * ldy + col, o);
    }
  }
}

// Persistent over rows: each wave takes rows wave_id, wave_id + waves_total,
// ...; per-lane dgamma partials live in registers and are combined per block
// through LDS into partial[blockIdx.x][n_cols].
template <typename T, typename W, int NCH>
__global__ __launch_bounds__(256) void men_bwd_k(
    const T* __restrict__ dy, const T* __restrict__ x, const W* __restrict__ w,
    const float* __restrict__ mu, T* __restrict__ dx, typename AccT<T>::type* __restrict__ partial,
    int64_t n_rows, int n_cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  __shared__ A red[kRowWaves][64 * V];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  A wv[NCH][V], dg[NCH][V];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * V;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      wv[c][i] = col < n_cols ? (A)w[col + i] : A(0);
      dg[c][i] = A(0);
    }
  }
  const A e = A(eps);
  for (int64_t row = (int64_t)blockIdx.x * kRowWaves + wave; row < n_rows;
       row += (int64_t)gridDim.x * kRowWaves) {
    VecT<T, V> ry[NCH], rx[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int col = (c * 64 + lane) * V;
      const bool in = col < n_cols;
      ry[c] = in ? ld_vec<T, V>(dy + row * lddy + col) : zero_vec<T, V>();
      rx[c] = in ? ld_vec<T, V>(x + row * ldx + col) : zero_vec<T, V>();
    }
    const A inv = A(1) / ((A)mu[row] + e);  // fused_ops.py:389-390
    A cs = A(0);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < V; ++i)
        cs += to_acc(ry[c].v[i]) * (to_acc(rx[c].v[i]) * inv * wv[c][i]);  // :404-405
    cs = wave_sum(cs);
    const A corr = cs / A(n_cols);  // fused_ops.py:408
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int col = (c * 64 + lane) * V;
      VecT<T, V> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A yy = to_acc(ry[c].v[i]);
        const A xx = to_acc(rx[c].v[i]);
        o.v[i] = from_acc<T>(yy * wv[c][i] * inv - sign_of(xx) * corr * inv);  // :418-421
        dg[c][i] += yy * (xx * inv);  // fused_ops.py:595-597
      }
      if (col < n_cols) st_vec<T, V>(dx + row * lddx + col, o);
    }
  }
  // Combine the 4 waves' partials chunk by chunk (fixed order).
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < V; ++i) red[wave][lane * V + i] = dg[c][i];
    __syncthreads();
    for (int t = threadIdx.x; t < 64 * V; t += blockDim.x) {
      const int col = c * 64 * V + t;
      if (col < n_cols) {
        A s = A(0);
#pragma unroll
        for (int ww = 0; ww < kRowWaves; ++ww) s += red[ww][t];
        partial[(int64_t)blockIdx.x * n_cols + col] = s;
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void men_fwd_mp_k(const T* __restrict__ x, const void* __restrict__ wp,
                                                    int w_is_f32, T* __restrict__ y,
                                                    float* __restrict__ mu, int64_t n_rows,
                                                    int n_cols, int64_t ldx, int64_t ldy,
                                                    float eps) {
  typedef typename AccT<T>::type A;
  __shared__ A sh[kRowWaves];
  const int64_t row = blockIdx.x;
  A s = A(0);
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) s += fabs(to_acc(x[row * ldx + c]));
  s = block_sum(s, sh);
  const A mean = s / A(n_cols);
  const A inv = A(1) / (mean + A(eps));
  if (threadIdx.x == 0) mu[row] = (float)mean;
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
    const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
    y[row * ldy + c] = from_acc<T>(to_acc(x[row * ldx + c]) * inv * wv);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void men_bwd_mp_k(
    const T* __restrict__ dy, const T* __restrict__ x, const void* __restrict__ wp, int w_is_f32,
    const float* __restrict__ mu, T* __restrict__ dx, typename AccT<T>::type* __restrict__ partial,
    int64_t n_rows, int n_cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps) {
  typedef typename AccT<T>::type A;
  __shared__ A sh[kRowWaves];
  A* part = partial + (int64_t)blockIdx.x * n_cols;  // owned by this block
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) part[c] = A(0);
  const A e = A(eps);
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const A inv = A(1) / ((A)mu[row] + e);
    A cs = A(0);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
      cs += to_acc(dy[row * lddy + c]) * (to_acc(x[row * ldx + c]) * inv * wv);
    }
    cs = block_sum(cs, sh);
    const A corr = cs / A(n_cols);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
      const A yy = to_acc(dy[row * lddy + c]);
      const A xx = to_acc(x[row * ldx + c]);
      dx[row * lddx + c] = from_acc<T>(yy * wv * inv - sign_of(xx) * corr * inv);
      part[c] += yy * (xx * inv);  // same thread owns column c throughout
    }
  }
}

// dw[c] = sum_g partial[g][c], fixed order: 16 waves stride over g, then the
// 16 wave sums are added in wave order.
template <typename A>
__global__ __launch_bounds__(1024) void colsum_k(const A* __restrict__ partial, int G, int n_cols,
                                                 A* __restrict__ out) {
  __shared__ A red[16][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  A s = A(0);
  if (col < n_cols)
    for (int g = wave; g < G; g += 16) s += partial[(int64_t)g * n_cols + col];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < n_cols) {
    A t = A(0);
#pragma unroll
    for (int ww = 0; ww < 16; ++ww) t += red[ww][lane];
    out[col] = t;
  }
}

template <typename A> __global__ void fill_zero_k(A* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = A(0);
}

// ============================================================================
// Host launchers
// ============================================================================

static inline int pick_nch(int64_t n_cols, int per) {
  const int64_t need = (n_cols + per - 1) / per;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  if (need <= 16) return 16;
  return 0;
}

#define KAT_NCH_SWITCH(nch, ...)          \
  switch (nch) {                          \
    case 1: { constexpr int N = 1; __VA_ARGS__; } break;  \
    case 2: { constexpr int N = 2; __VA_ARGS__; } break;  \
    case 4: { constexpr int N = 4; __VA_ARGS__; } break;  \
    case 8: { constexpr int N = 8; __VA_ARGS__; } break;  \
    default: { constexpr int N = 16; __VA_ARGS__; } break; \
  }

template <typename T>
static int swiglu_fwd_t(const T* g, const T* v, T* o, int64_t rows, int64_t cols, int64_t ldg,
                        int64_t ldv, int64_t ldo, hipStream_t st) {
  constexpr int V = Raw<T>::V;
  if (ldg == cols && ldv == cols && ldo == cols && (rows * cols) % V == 0 &&
      rows * cols / V <= kMaxChunks) {  // contiguous: one flat row
    cols = rows * cols;
    rows = 1;
    ldg = ldv = ldo = cols;
  }
  const bool vec = cols % V == 0 && ldg % V == 0 && ldv % V == 0 && ldo % V == 0 &&
                   aligned16(g) && aligned16(v) && aligned16(o) && cols / V <= kMaxChunks;
  if (vec) {
    const int64_t cpr = cols / V;
    const int64_t rows_per = std::max<int64_t>(1, kMaxChunks / cpr);
    for (int64_t r0 = 0; r0 < rows; r0 += rows_per) {
      const int64_t nr = std::min(rows_per, rows - r0);
      const uint32_t n_chunks = (uint32_t)(nr * cpr);
      const unsigned blocks = (n_chunks + kEwThreads * kEwUnroll - 1) / (kEwThreads * kEwUnroll);
      hipLaunchKernelGGL((swiglu_fwd_k<T, V>), dim3(blocks), dim3(kEwThreads), 0, st,
                         g + r0 * ldg, v + r0 * ldv, o + r0 * ldo, n_chunks, (uint32_t)cpr, ldg,
                         ldv, ldo);
    }
  } else {
    const uint64_t n = (uint64_t)rows * (uint64_t)cols;
    const uint64_t blocks = std::min<uint64_t>((n + kEwThreads - 1) / kEwThreads, 65536);
    hipLaunchKernelGGL((swiglu_fwd_scalar_k<T>), dim3((unsigned)blocks), dim3(kEwThreads), 0, st,
                       g, v, o, n, (uint64_t)cols, ldg, ldv, ldo);
  }
  return check_launch("kat_rswiglu_fwd");
}

template <typename T>
static int swiglu_bwd_t(const T* dy, const T* g, const T* v, T* dg, T* dv, int64_t rows,
                        int64_t cols, int64_t lddy, int64_t ldg, int64_t ldv, int64_t lddg,
                        int64_t lddv, hipStream_t st) {
  constexpr int V = Raw<T>::V;
  if (lddy == cols && ldg == cols && ldv == cols && lddg == cols && lddv == cols &&
      (rows * cols) % V == 0 && rows * cols / V <= kMaxChunks) {  // contiguous: one flat row
    cols = rows * cols;
    rows = 1;
    lddy = ldg = ldv = lddg = lddv = cols;
  }
  const bool vec = cols % V == 0 && lddy % V == 0 && ldg % V == 0 && ldv % V == 0 &&
                   lddg % V == 0 && lddv % V == 0 && aligned16(dy) && aligned16(g) &&
                   aligned16(v) && aligned16(dg) && aligned16(dv) && cols / V <= kMaxChunks;
  if (vec) {
    const int64_t cpr = cols / V;
    const int64_t rows_per = std::max<int64_t>(1, kMaxChunks / cpr);
    for (int64_t r0 = 0; r0 < rows; r0 += rows_per) {
      const int64_t nr = std::min(rows_per, rows - r0);
      const uint32_t n_chunks = (uint32_t)(nr * cpr);
      const unsigned blocks = (n_chunks + kEwThreads * kEwUnroll - 1) / (kEwThreads * kEwUnroll);
      hipLaunchKernelGGL((swiglu_bwd_k<T, V>), dim3(blocks), dim3(kEwThreads), 0, st,
                         dy + r0 * lddy, g + r0 * ldg, v + r0 * ldv, dg + r0 * lddg,
                         dv + r0 * lddv, n_chunks, (uint32_t)cpr, lddy, ldg, ldv, lddg, lddv);
    }
  } else {
    const uint64_t n = (uint64_t)rows * (uint64_t)cols;
    const uint64_t blocks = std::min<uint64_t>((n + kEwThreads - 1) / kEwThreads, 65536);
    hipLaunchKernelGGL((swiglu_bwd_scalar_k<T>), dim3((unsigned)blocks), dim3(kEwThreads), 0, st,
                       dy, g, v, dg, dv, n, (uint64_t)cols, lddy, ldg, ldv, lddg, lddv);
  }
  return check_launch("kat_rswiglu_bwd");
}

template <typename T>
static int rsoftmax_fwd_t(const T* x, T* p, int64_t rows, int64_t cols, int64_t ldx, int64_t ldp,
                          float eps, hipStream_t st) {
  constexpr int V = Raw<T>::V;
  const bool vec = cols % V == 0 && ldx % V == 0 && ldp % V == 0 && aligned16(x) && aligned16(p);
  const int nch = vec ? pick_nch(cols, 64 * V) : 0;
  if (nch) {
    const int64_t blocks = (rows + kRowWaves - 1) / kRowWaves;
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((rsoftmax_fwd_k<T, N>), dim3((unsigned)blocks),
                                           dim3(256), 0, st, x, p, rows, (int)cols, ldx, ldp, eps));
  } else {
    hipLaunchKernelGGL((rsoftmax_fwd_mp_k<T>), dim3((unsigned)rows), dim3(256), 0, st, x, p, rows,
                       (int)cols, ldx, ldp, eps);
  }
  return check_launch("kat_rsoftmax_fwd");
}

template <typename T>
static int rsoftmax_bwd_t(const T* dy, const T* x, const T* p, T* dx, int64_t rows, int64_t cols,
                          int64_t lddy, int64_t ldx, int64_t ldp, int64_t lddx, float eps,
                          hipStream_t st) {
  constexpr int V = Raw<T>::V;
  const bool vec = cols % V == 0 && lddy % V == 0 && ldx % V == 0 && ldp % V == 0 &&
                   lddx % V == 0 && aligned16(dy) && aligned16(x) && aligned16(p) && aligned16(dx);
  const int nch = vec ? pick_nch(cols, 64 * V) : 0;
  if (nch) {
    const int64_t blocks = (rows + kRowWaves - 1) / kRowWaves;
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((rsoftmax_bwd_k<T, N>), dim3((unsigned)blocks),
                                           dim3(256), 0, st, dy, x, p, dx, rows, (int)cols, lddy,
                                           ldx, ldp, lddx, eps));
  } else {
    hipLaunchKernelGGL((rsoftmax_bwd_mp_k<T>), dim3((unsigned)rows), dim3(256), 0, st, dy, x, p,
                       dx, rows, (int)cols, lddy, ldx, ldp, lddx, eps);
  }
  return check_launch("kat_rsoftmax_bwd");
}

template <typename T, typename W>
static int men_fwd_t(const T* x, const W* w, T* y, float* mu, int64_t rows, int64_t cols,
                     int64_t ldx, int64_t ldy, float eps, hipStream_t st) {
  constexpr int V = Raw<T>::V;
  const bool vec = cols % V == 0 && ldx % V == 0 && ldy % V == 0 && aligned16(x) && aligned16(y);
  const int nch = vec ? pick_nch(cols, 64 * V) : 0;
  if (nch) {
    const int64_t blocks = (rows + kRowWaves - 1) / kRowWaves;
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((men_fwd_k<T, W, N>), dim3((unsigned)blocks), dim3(256),
                                           0, st, x, w, y, mu, rows, (int)cols, ldx, ldy, eps));
  } else {
    hipLaunchKernelGGL((men_fwd_mp_k<T>), dim3((unsigned)rows), dim3(256), 0, st, x,
                       (const void*)w, (int)std::is_same<W, float>::value, y, mu, rows, (int)cols,
                       ldx, ldy, eps);
  }
  return check_launch("kat_men_fwd");
}

static int men_bwd_grid(int64_t rows, bool resident) {
  const int64_t want = resident ? (rows + kRowWaves - 1) / kRowWaves : rows;
  const int64_t cap = 2LL * num_cus();
  return (int)std::max<int64_t>(1, std::min<int64_t>(want, cap));
}

template <typename T, typename W>
static int men_bwd_t(const T* dy, const T* x, const W* w, const float* mu, T* dx,
                     typename AccT<T>::type* dw, void* ws, size_t ws_bytes, int64_t rows,
                     int64_t cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps,
                     hipStream_t st) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  const bool vec = cols % V == 0 && lddy % V == 0 && ldx % V == 0 && lddx % V == 0 &&
                   aligned16(dy) && aligned16(x) && aligned16(dx);
  const int nch = vec ? pick_nch(cols, 64 * V) : 0;
  const int G = men_bwd_grid(rows, nch != 0);
  const size_t need = (size_t)G * (size_t)cols * sizeof(A);
  if (ws_bytes < need || (need && ws == nullptr))
    return fail(KAT_EINVAL, "kat_men_bwd: workspace %zu bytes < required %zu", ws_bytes, need);
  A* partial = reinterpret_cast<A*>(ws);
  if (nch) {
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((men_bwd_k<T, W, N>), dim3(G), dim3(256), 0, st, dy, x,
                                           w, mu, dx, partial, rows, (int)cols, lddy, ldx, lddx,
                                           eps));
  } else {
    hipLaunchKernelGGL((men_bwd_mp_k<T>), dim3(G), dim3(256), 0, st, dy, x, (const void*)w,
                       (int)std::is_same<W, float>::value, mu, dx, partial, rows, (int)cols, lddy, ldx, lddx, eps);
  }
  int rc = check_launch("kat_men_bwd");
  if (rc) return rc;
  hipLaunchKernelGGL((colsum_k<A>), dim3((unsigned)((cols + 63) / 64)), dim3(1024), 0, st,
                     partial, G, (int)cols, dw);
  return check_launch("kat_men_bwd (dw reduction)");
}

}  // namespace kat

// ============================================================================
// C ABI
// ============================================================================

using namespace kat;

#define KAT_DISPATCH_T(dtype, name, ...)                                              \
  switch (dtype) {                                                                    \
    case KAT_F32: { typedef float T; return __VA_ARGS__; }                            \
    case KAT_BF16: { typedef bf16 T; return __VA_ARGS__; }                            \
    case KAT_F16: { typedef f16 T; return __VA_ARGS__; }                              \
    case KAT_F64: { typedef double T; return __VA_ARGS__; }                           \
    default: return fail(KAT_EUNSUPPORTED, "%s: unsupported dtype %d", name, (int)dtype); \
  }

static int check_rows(const char* name, int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return fail(KAT_EINVAL, "%s: negative size", name);
  if (cols > 0x7fffffffLL) return fail(KAT_EUNSUPPORTED, "%s: n_cols too large", name);
  if (rows > 0x7fffffffLL * (int64_t)kRowWaves)
    return fail(KAT_EUNSUPPORTED, "%s: n_rows too large", name);
  return KAT_OK;
}

static int check_ld(const char* name, int64_t cols, std::initializer_list<int64_t> lds) {
  for (int64_t ld : lds)
    if (ld < cols) return fail(KAT_EINVAL, "%s: leading dimension %lld < n_cols %lld", name,
                               (long long)ld, (long long)cols);
  return KAT_OK;
}

extern "C" int kat_rswiglu_fwd(const void* gate, const void* value, void* out, int64_t n_rows,
                               int64_t n_cols, int64_t ld_gate, int64_t ld_value, int64_t ld_out,
                               int dtype, void* stream) {
  const char* nm = "kat_rswiglu_fwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!gate || !value || !out) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_gate, ld_value, ld_out})) return rc;
  KAT_DISPATCH_T(dtype, nm,
                 swiglu_fwd_t<T>((const T*)gate, (const T*)value, (T*)out, n_rows, n_cols, ld_gate,
                                 ld_value, ld_out, as_stream(stream)));
}

extern "C" int kat_rswiglu_bwd(const void* dy, const void* gate, const void* value, void* dgate,
                               void* dvalue, int64_t n_rows, int64_t n_cols, int64_t ld_dy,
                               int64_t ld_gate, int64_t ld_value, int64_t ld_dgate,
                               int64_t ld_dvalue, int dtype, void* stream) {
  const char* nm = "kat_rswiglu_bwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!dy || !gate || !value || !dgate || !dvalue) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_dy, ld_gate, ld_value, ld_dgate, ld_dvalue})) return rc;
  KAT_DISPATCH_T(dtype, nm,
                 swiglu_bwd_t<T>((const T*)dy, (const T*)gate, (const T*)value, (T*)dgate,
                                 (T*)dvalue, n_rows, n_cols, ld_dy, ld_gate, ld_value, ld_dgate,
                                 ld_dvalue, as_stream(stream)));
}

extern "C" int kat_rsoftmax_fwd(const void* x, void* p, int64_t n_rows, int64_t n_cols,
                                int64_t ld_x, int64_t ld_p, float eps, int dtype, void* stream) {
  const char* nm = "kat_rsoftmax_fwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!x || !p) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_x, ld_p})) return rc;
  KAT_DISPATCH_T(dtype, nm,
                 rsoftmax_fwd_t<T>((const T*)x, (T*)p, n_rows, n_cols, ld_x, ld_p, eps,
                                   as_stream(stream)));
}

extern "C" int kat_rsoftmax_bwd(const void* dy, const void* x, const void* p, void* dx,
                                int64_t n_rows, int64_t n_cols, int64_t ld_dy, int64_t ld_x,
                                int64_t ld_p, int64_t ld_dx, float eps, int dtype, void* stream) {
  const char* nm = "kat_rsoftmax_bwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!dy || !x || !p || !dx) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_dy, ld_x, ld_p, ld_dx})) return rc;
  KAT_DISPATCH_T(dtype, nm,
                 rsoftmax_bwd_t<T>((const T*)dy, (const T*)x, (const T*)p, (T*)dx, n_rows, n_cols,
                                   ld_dy, ld_x, ld_p, ld_dx, eps, as_stream(stream)));
}

extern "C" int kat_men_fwd(const void* x, const void* w, void* y, float* mu, int64_t n_rows,
                           int64_t n_cols, int64_t ld_x, int64_t ld_y, float eps, int dtype,
                           int dtype_w, void* stream) {
  const char* nm = "kat_men_fwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!x || !w || !y || !mu) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_x, ld_y})) return rc;
  const hipStream_t st = as_stream(stream);
  if (dtype_w == dtype) {
    KAT_DISPATCH_T(dtype, nm,
                   (men_fwd_t<T, T>((const T*)x, (const T*)w, (T*)y, mu, n_rows, n_cols, ld_x, ld_y,
                                    eps, st)));
  }
  if (dtype_w == KAT_F32 && dtype != KAT_F64) {
    KAT_DISPATCH_T(dtype, nm,
                   (men_fwd_t<T, float>((const T*)x, (const float*)w, (T*)y, mu, n_rows, n_cols,
                                        ld_x, ld_y, eps, st)));
  }
  return fail(KAT_EUNSUPPORTED, "%s: weight dtype %d with input dtype %d", nm, dtype_w, dtype);
}

extern "C" size_t kat_men_bwd_workspace_size(int64_t n_rows, int64_t n_cols, int dtype) {
  const int sz = dtype_size(dtype);
  if (n_rows <= 0 || n_cols <= 0 || sz == 0) return 0;
  // alignment decides between the two kernels at call time: size for the larger grid
  const int G = std::max(men_bwd_grid(n_rows, true), men_bwd_grid(n_rows, false));
  const size_t acc = dtype == KAT_F64 ? 8 : 4;
  return (size_t)G * (size_t)n_cols * acc;
}

extern "C" int kat_men_bwd(const void* dy, const void* x, const void* w, const float* mu, void* dx,
                           void* dw, void* workspace, size_t workspace_bytes, int64_t n_rows,
                           int64_t n_cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, float eps,
                           int dtype, int dtype_w, void* stream) {
  const char* nm = "kat_men_bwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_cols == 0) return KAT_OK;
  if (!dw) return fail(KAT_EINVAL, "%s: null pointer", nm);
  const hipStream_t st = as_stream(stream);
  if (n_rows == 0) {  // no rows: dw = 0 (a fill kernel, not a memset node)
    if (dtype == KAT_F64)
      hipLaunchKernelGGL((fill_zero_k<double>), dim3((unsigned)((n_cols + 255) / 256)), dim3(256),
                         0, st, (double*)dw, n_cols);
    else
      hipLaunchKernelGGL((fill_zero_k<float>), dim3((unsigned)((n_cols + 255) / 256)), dim3(256),
                         0, st, (float*)dw, n_cols);
    return check_launch(nm);
  }
  if (!dy || !x || !w || !mu || !dx) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_dy, ld_x, ld_dx})) return rc;
  if (dtype_w == dtype) {
    KAT_DISPATCH_T(dtype, nm,
                   (men_bwd_t<T, T>((const T*)dy, (const T*)x, (const T*)w, mu, (T*)dx,
                                    (typename AccT<T>::type*)dw, workspace, workspace_bytes,
                                    n_rows, n_cols, ld_dy, ld_x, ld_dx, eps, st)));
  }
  if (dtype_w == KAT_F32 && dtype != KAT_F64) {
    KAT_DISPATCH_T(dtype, nm,
                   (men_bwd_t<T, float>((const T*)dy, (const T*)x, (const float*)w, mu, (T*)dx,
                                        (typename AccT<T>::type*)dw, workspace, workspace_bytes,
                                        n_rows, n_cols, ld_dy, ld_x, ld_dx, eps, st)));
  }
  return fail(KAT_EUNSUPPORTED, "%s: weight dtype %d with input dtype %d", nm, dtype_w, dtype);
}
