// Bandwidth-bound row operations of the algebraic transformer on gfx950:
// rational softmax, rational SwiGLU and mean-error norm, forward and backward.
//
// Design (MI355X): these ops do a handful of flops per byte, so the only
// roofline that matters is HBM (8 TB/s). Every kernel touches each tensor
// exactly once:
//   * row-resident kernels (softmax, norm): a 256-thread block owns a row at a
//     time, holds it in registers as packed 16-byte vectors, reduces with
//     wavefront shuffles plus a 4-entry LDS exchange and writes the result --
//     one HBM pass where the reference makes two (fused_ops.py:74-106,
//     319-342, 395-423);
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

// Streaming 16-byte accesses. Every tensor is read once per kernel, so loads
// are non-temporal; stores are plain. Measured on the MI355X with cold caches
// at the norm's size (128 MiB per tensor): a copy with non-temporal loads and
// plain stores runs 1 read + 1 write in 43.8 us and 2 reads + 1 write in
// 61.8 us, against 46.2 / 64.7 us with non-temporal stores and 47.5 / 69.9 us
// with plain loads; the norm, residual-norm and SwiGLU steps gain 2-7% from the
// plain stores, the softmax step 3%.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
template <typename T, int V>
__device__ __forceinline__ VecT<T, V> ld_vec(const T* __restrict__ p) {
  static_assert(sizeof(VecT<T, V>) == 16, "16-byte vectors");
  const u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return __builtin_bit_cast(VecT<T, V>, r);
}
template <typename T, int V>
__device__ __forceinline__ void st_vec(T* __restrict__ p, const VecT<T, V>& v) {
  *reinterpret_cast<u32x4_t*>(p) = __builtin_bit_cast(u32x4_t, v);
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

// The norm backward's per-element terms with every fused multiply-add written
// out, so the rounding does not depend on which products the compiler
// contracts in a given template instance: the plain, residual-fused and
// narrow-dy kernels, single- and multi-pass, all round identically.
//   dx = dy * (w * inv) - sign(x) * corr * inv     (fused_ops.py:418-421)
template <typename A>
__device__ __forceinline__ A men_dx(A yy, A xx, A wv, A inv, A corr) {
  return __builtin_fma(yy, wv * inv, -(sign_of(xx) * corr * inv));
}
template <>
__device__ __forceinline__ float men_dx<float>(float yy, float xx, float wv, float inv, float corr) {
  return __builtin_fmaf(yy, wv * inv, -(sign_of(xx) * corr * inv));
}
// v narrowed to Y (bf16 / fp16 from fp32) by a plain conversion of the
// rounded fp32 register value. Without the empty asm the compiler may fold the
// narrowing into the multiply that produced v (a mixed-precision FMA rounding
// the exact product once to fp16), which differs from the fp32 result followed
// by torch's cast in the last bit now and then; the narrow-output kernels must
// equal that cast.
template <typename Y, typename A> __device__ __forceinline__ Y narrow_to(A v) {
  if constexpr (sizeof(Y) < sizeof(A)) asm("" : "+v"(v));
  return from_acc<Y>(v);
}
//   acc + dy * p     (row sum of dy * y_hat; column sum of dy * x_hat)
template <typename A> __device__ __forceinline__ A men_fma(A yy, A p, A acc) {
  return __builtin_fma(yy, p, acc);
}
template <> __device__ __forceinline__ float men_fma<float>(float yy, float p, float acc) {
  return __builtin_fmaf(yy, p, acc);
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

// Row and column of 16-byte chunk cc (cpr chunks per row). A launch over one
// flat row (contiguous tensors) skips the integer division, which costs more
// VALU work than the rest of the element math here (measured 5% of the
// forward's time), and a power-of-two row length (the model's packed gate /
// value halves) shifts instead; the branches are uniform across the grid.
__device__ __forceinline__ void chunk_rc(uint32_t cc, uint32_t cpr, uint32_t n_chunks, int V,
                                         int64_t& row, int64_t& col) {
  if (cpr >= n_chunks) {
    row = 0;
    col = (int64_t)cc * V;
  } else if ((cpr & (cpr - 1u)) == 0u) {
    row = (int64_t)(cc >> __builtin_ctz(cpr));
    col = (int64_t)(cc & (cpr - 1u)) * V;
  } else {
    const uint32_t r = cc / cpr;
    row = (int64_t)r;
    col = (int64_t)(cc - r * cpr) * V;
  }
}

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
    chunk_rc(cc, cpr, n_chunks, V, row[u], col[u]);
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
        out.v[i] = from_acc<T>(gg * rsig_t<T>(gg) * vv);  // fused_ops.py:224-227
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
    chunk_rc(cc, cpr, n_chunks, V, row[u], col[u]);
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
        const A sig = A(0.5) * (ediv<T>(gg, den) + A(1));
        const A sd = ediv<T>(A(0.5), den * den);
        ov.v[i] = from_acc<T>(y * gg * sig);
        og.v[i] = from_acc<T>(y * vv * (sig + gg * sd));
      }
      st_vec<T, V>(dg + row[u] * lddg + col[u], og);
      st_vec<T, V>(dv + row[u] * lddv + col[u], ov);
    }
  }
}

// Scalar fallback for misaligned / odd-width inputs (e.g. the packed gate /
// value halves of an odd d_ffn, whose value half is only 2-byte aligned). A 2D
// grid: blockIdx.y walks rows, x and the unrolled lanes walk columns, so no
// element index is divided by the row length (a 64-bit division per element
// cost more than the memory traffic); each thread keeps kEwUnroll elements in
// flight, 256 columns apart, for coalesced 2-byte accesses.
template <typename T>
__global__ __launch_bounds__(kEwThreads) void swiglu_fwd_scalar_k(
    const T* __restrict__ g, const T* __restrict__ v, T* __restrict__ o, int64_t rows,
    int64_t cols, int64_t ldg, int64_t ldv, int64_t ldo) {
  typedef typename AccT<T>::type A;
  const int64_t c0 = (int64_t)blockIdx.x * (kEwThreads * kEwUnroll) + threadIdx.x;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    T gr[kEwUnroll], vr[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
      const int64_t c = c0 + u * kEwThreads;
      const int64_t cc = c < cols ? c : 0;
      gr[u] = g[r * ldg + cc];
      vr[u] = v[r * ldv + cc];
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
      const int64_t c = c0 + u * kEwThreads;
      const A gg = to_acc(gr[u]), vv = to_acc(vr[u]);
      if (c < cols) o[r * ldo + c] = from_acc<T>(gg * rsig_t<T>(gg) * vv);  // fused_ops.py:224-227
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kEwThreads) void swiglu_bwd_scalar_k(
    const T* __restrict__ dy, const T* __restrict__ g, const T* __restrict__ v,
    T* __restrict__ dg, T* __restrict__ dv, int64_t rows, int64_t cols, int64_t lddy, int64_t ldg,
    int64_t ldv, int64_t lddg, int64_t lddv) {
  typedef typename AccT<T>::type A;
  const int64_t c0 = (int64_t)blockIdx.x * (kEwThreads * kEwUnroll) + threadIdx.x;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    T yr[kEwUnroll], gr[kEwUnroll], vr[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
      const int64_t c = c0 + u * kEwThreads;
      const int64_t cc = c < cols ? c : 0;
      yr[u] = dy[r * lddy + cc];
      gr[u] = g[r * ldg + cc];
      vr[u] = v[r * ldv + cc];
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
      const int64_t c = c0 + u * kEwThreads;
      const A y = to_acc(yr[u]), gg = to_acc(gr[u]), vv = to_acc(vr[u]);
      const A den = fabs(gg) + A(1);  // fused_ops.py:276-285
      const A sig = A(0.5) * (ediv<T>(gg, den) + A(1));
      const A sd = ediv<T>(A(0.5), den * den);
      if (c < cols) {
        dv[r * lddv + c] = from_acc<T>(y * gg * sig);
        dg[r * lddg + c] = from_acc<T>(y * vv * (sig + gg * sd));
      }
    }
  }
}

// 2D grid of the scalar SwiGLU kernels: column blocks by row blocks (rows are
// walked in a loop past 65535)
static dim3 scalar_grid(int64_t rows, int64_t cols) {
  const int64_t per = (int64_t)kEwThreads * kEwUnroll;
  return dim3((unsigned)((cols + per - 1) / per), (unsigned)std::min<int64_t>(rows, 65535));
}

// ============================================================================
// rational softmax -- fused_ops.py:52-189
// ============================================================================

// Row-resident kernels: a 256-thread block owns one row at a time and each
// thread a fixed column slice (16-byte chunks tid, tid + 256, ...), so per-row
// reductions are one wave reduction plus a 4-entry LDS exchange. Blocks are
// persistent over rows (row = blockIdx.x + i * gridDim.x) and keep the next
// two rows' loads in flight while the current one is reduced and written,
// which keeps HBM busy without relying on occupancy alone.

// Block-wide sum for 256 threads; `par` alternates per row so consecutive rows
// use different LDS slots and one barrier per row suffices.
template <typename A> __device__ __forceinline__ A block_sum_par(A v, A (*red)[kRowWaves], int par) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[par][threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[par][0] + red[par][1]) + (red[par][2] + red[par][3]);
}

// Loads this thread's chunks of one row. Chunks past the row end re-read the
// row's first chunk (always in bounds) and are masked where they are used:
// a conditional load here would compile to a branch that waits for the data
// on the spot, serialising the prefetch.
// FULL: the row is exactly NCH chunk rounds long, so every chunk is in range
// and the column tests fold away (the norm kernels take this when it holds).
template <typename T, int NCH, bool FULL = false>
__device__ __forceinline__ void load_row(const T* __restrict__ base, int n_cols, VecT<T, Raw<T>::V> (&r)[NCH]) {
  constexpr int V = Raw<T>::V;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = ((int)threadIdx.x + 256 * k) * V;
    r[k] = ld_vec<T, V>(base + ((FULL || col < n_cols) ? col : 0));
  }
}
template <bool FULL = false> __device__ __forceinline__ bool chunk_in(int k, int V, int n_cols) {
  return FULL || ((int)threadIdx.x + 256 * k) * V < n_cols;
}

// The weight values of this thread's chunks, with 16-byte loads (the caller
// checks 16-byte alignment of w); out-of-row chunks read chunk 0.
template <typename T, typename W, int NCH>
__device__ __forceinline__ void load_weight(const W* __restrict__ w, int n_cols,
                                            typename AccT<T>::type (&wv)[NCH][Raw<T>::V]) {
  constexpr int V = Raw<T>::V;
  constexpr int PER = 16 / (int)sizeof(W);  // weights per 16-byte load
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = ((int)threadIdx.x + 256 * k) * V;
    const W* base = w + (col < n_cols ? col : 0);
    if constexpr (V % PER == 0) {
#pragma unroll
      for (int j = 0; j < V / PER; ++j) {
        const VecT<W, PER> r = *reinterpret_cast<const VecT<W, PER>*>(base + j * PER);
#pragma unroll
        for (int e = 0; e < PER; ++e) wv[k][j * PER + e] = (typename AccT<T>::type)r.v[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) wv[k][e] = (typename AccT<T>::type)base[e];
    }
  }
}

// g = 2 / ((|x| + 1)^2 (sigma(x) + eps)), the softmax backward's derivative
// factor (fused_ops.py:179-187). With den = |x| + 1, sigma(x) + eps =
// (0.5 (x + den) + eps den) / den, so g = 2 / (den (0.5 (x + den) + eps den)):
// one reciprocal for bf16 / fp16 data; fp32 / fp64 data keep the reference's
// form with IEEE divides.
template <typename T, typename A> __device__ __forceinline__ A rsm_g(A x, A e) {
  const A den = fabs(x) + A(1);
  if constexpr (sizeof(T) == 2 && sizeof(A) == 4) {
    return A(2) * __builtin_amdgcn_rcpf(den * fmaf(e, den, A(0.5) * (x + den)));
  } else {
    const A sig = A(0.5) * (x / den + A(1));
    return A(2) / (den * den * (sig + e));
  }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void rsoftmax_fwd_k(const T* __restrict__ x, T* __restrict__ p,
                                                      int64_t n_rows, int n_cols, int64_t ldx,
                                                      int64_t ldp, float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  __shared__ A red[2][kRowWaves];
  const int64_t G = gridDim.x;
  int64_t row = blockIdx.x;
  // rows `row`, `row + G` in flight; rows past the end clamp to the last row
  // (loaded, never used) so no load sits behind a branch
  const int64_t last = n_rows - 1;
  VecT<T, V> cur[NCH], nx1[NCH];
  load_row<T, NCH>(x + std::min(row, last) * ldx, n_cols, cur);
  load_row<T, NCH>(x + std::min(row + G, last) * ldx, n_cols, nx1);
  for (int par = 0; row < n_rows; row += G, par ^= 1) {
    VecT<T, V> nx2[NCH];
    load_row<T, NCH>(x + std::min(row + 2 * G, last) * ldx, n_cols, nx2);
    A f[NCH][V];
    A sum = A(0);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const bool in = ((int)threadIdx.x + 256 * k) * V < n_cols;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A sg = rsig_t<T>(to_acc(cur[k].v[i]));  // fused_ops.py:81-86
        const A s2 = sg * sg;
        f[k][i] = s2 * s2;
        sum += in ? f[k][i] : A(0);
      }
    }
    sum = block_sum_par(sum, red, par);
    const A inv = A(1) / (sum + A(eps));  // fused_ops.py:90
    T* pr = p + row * ldp;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int col = ((int)threadIdx.x + 256 * k) * V;
      if (col < n_cols) {
        VecT<T, V> o;
#pragma unroll
        for (int i = 0; i < V; ++i) o.v[i] = from_acc<T>(f[k][i] * inv);  // fused_ops.py:104
        st_vec<T, V>(pr + col, o);
      }
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      cur[k] = nx1[k];
      nx1[k] = nx2[k];
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
  __shared__ A red[2][kRowWaves];
  const int64_t G = gridDim.x;
  int64_t row = blockIdx.x;
  const int64_t last = n_rows - 1;
  VecT<T, V> cy[NCH], cp[NCH], cx[NCH], y1[NCH], p1[NCH], x1[NCH];
  {
    const int64_t r0 = std::min(row, last), r1 = std::min(row + G, last);
    load_row<T, NCH>(dy + r0 * lddy, n_cols, cy);
    load_row<T, NCH>(p + r0 * ldp, n_cols, cp);
    load_row<T, NCH>(x + r0 * ldx, n_cols, cx);
    load_row<T, NCH>(dy + r1 * lddy, n_cols, y1);
    load_row<T, NCH>(p + r1 * ldp, n_cols, p1);
    load_row<T, NCH>(x + r1 * ldx, n_cols, x1);
  }
  const A e = A(eps);
  for (int par = 0; row < n_rows; row += G, par ^= 1) {
    VecT<T, V> ny[NCH], np[NCH], nx[NCH];
    {
      const int64_t r2 = std::min(row + 2 * G, last);
      load_row<T, NCH>(dy + r2 * lddy, n_cols, ny);
      load_row<T, NCH>(p + r2 * ldp, n_cols, np);
      load_row<T, NCH>(x + r2 * ldx, n_cols, nx);
    }
    A dot = A(0);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const bool in = chunk_in(k, V, n_cols);
#pragma unroll
      for (int i = 0; i < V; ++i) dot += in ? to_acc(cy[k].v[i]) * to_acc(cp[k].v[i]) : A(0);  // :167
    }
    dot = block_sum_par(dot, red, par);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int col = ((int)threadIdx.x + 256 * k) * V;
      if (col < n_cols) {
        VecT<T, V> o;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const A xx = to_acc(cx[k].v[i]);
          const A g = rsm_g<T>(xx, e);  // fused_ops.py:179-187
          o.v[i] = from_acc<T>(to_acc(cp[k].v[i]) * g * (to_acc(cy[k].v[i]) - dot));
        }
        st_vec<T, V>(dx + row * lddx + col, o);
      }
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      cy[k] = y1[k];
      cp[k] = p1[k];
      cx[k] = x1[k];
      y1[k] = ny[k];
      p1[k] = np[k];
      x1[k] = nx[k];
    }
  }
}

// One wave per row: for few rows (at most 16 per CU, one residency round), a
// wave loads its whole row at once, reduces it with cross-lane operations only
// (no LDS, no barrier) and writes it. The persistent block kernels above
// pipeline rows within a block, which pays off only when each block gets many
// rows; at 4096 rows of 4096 this is 6-12% faster. Lane l owns the 16-byte
// chunks l, l + 64, ...; chunks past the row end re-read chunk 0 and are
// masked, as in load_row.
template <typename T, int NCH>
__device__ __forceinline__ void load_row_w(const T* __restrict__ base, int lane, int n_cols,
                                           VecT<T, Raw<T>::V> (&r)[NCH]) {
  constexpr int V = Raw<T>::V;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = (lane + 64 * k) * V;
    r[k] = ld_vec<T, V>(base + (col < n_cols ? col : 0));
  }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void rsoftmax_fwd_w_k(const T* __restrict__ x, T* __restrict__ p,
                                                        int64_t n_rows, int n_cols, int64_t ldx,
                                                        int64_t ldp, float eps) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // the whole wave leaves; nothing below synchronises
  VecT<T, V> cur[NCH];
  load_row_w<T, NCH>(x + row * ldx, lane, n_cols, cur);
  A f[NCH][V];
  A sum = A(0);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const bool in = (lane + 64 * k) * V < n_cols;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const A sg = rsig_t<T>(to_acc(cur[k].v[i]));  // fused_ops.py:81-86
      const A s2 = sg * sg;
      f[k][i] = s2 * s2;
      sum += in ? f[k][i] : A(0);
    }
  }
  sum = wave_sum(sum);
  const A inv = A(1) / (sum + A(eps));  // fused_ops.py:90
  // every output vector is formed before the first store, so no VALU result
  // lands in a register that a 16-byte store has just read
  VecT<T, V> o[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int i = 0; i < V; ++i) o[k].v[i] = from_acc<T>(f[k][i] * inv);  // fused_ops.py:104
  T* pr = p + row * ldp;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = (lane + 64 * k) * V;
    if (col < n_cols) st_vec<T, V>(pr + col, o[k]);
  }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void rsoftmax_bwd_w_k(const T* __restrict__ dy,
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
  VecT<T, V> cy[NCH], cp[NCH], cx[NCH];
  load_row_w<T, NCH>(dy + row * lddy, lane, n_cols, cy);
  load_row_w<T, NCH>(p + row * ldp, lane, n_cols, cp);
  load_row_w<T, NCH>(x + row * ldx, lane, n_cols, cx);
  A dot = A(0);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const bool in = (lane + 64 * k) * V < n_cols;
#pragma unroll
    for (int i = 0; i < V; ++i) dot += in ? to_acc(cy[k].v[i]) * to_acc(cp[k].v[i]) : A(0);  // :167
  }
  dot = wave_sum(dot);
  const A e = A(eps);
  VecT<T, V> o[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const A xx = to_acc(cx[k].v[i]);
      const A g = rsm_g<T>(xx, e);  // fused_ops.py:179-187
      o[k].v[i] = from_acc<T>(to_acc(cp[k].v[i]) * g * (to_acc(cy[k].v[i]) - dot));
    }
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = (lane + 64 * k) * V;
    if (col < n_cols) st_vec<T, V>(dx + row * lddx + col, o[k]);
  }
}

// Multi-pass block-per-row fallbacks (wide rows, misaligned or odd widths);
// grid-stride over rows.
template <typename T>
__global__ __launch_bounds__(256) void rsoftmax_fwd_mp_k(const T* __restrict__ x,
                                                         T* __restrict__ p, int64_t n_rows,
                                                         int n_cols, int64_t ldx, int64_t ldp,
                                                         float eps) {
  typedef typename AccT<T>::type A;
  __shared__ A sh[kRowWaves];
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const T* xr = x + row * ldx;
    A sum = A(0);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A s = rsig_t<T>(to_acc(xr[c]));
      const A s2 = s * s;
      sum += s2 * s2;
    }
    sum = block_sum(sum, sh);
    const A inv = A(1) / (sum + A(eps));
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A s = rsig_t<T>(to_acc(xr[c]));
      const A s2 = s * s;
      p[row * ldp + c] = from_acc<T>(s2 * s2 * inv);
    }
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
  const A e = A(eps);
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    A dot = A(0);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x)
      dot += to_acc(dy[row * lddy + c]) * to_acc(p[row * ldp + c]);
    dot = block_sum(dot, sh);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A xx = to_acc(x[row * ldx + c]);
      const A g = rsm_g<T>(xx, e);  // fused_ops.py:179-187
      dx[row * lddx + c] =
          from_acc<T>(to_acc(p[row * ldp + c]) * g * (to_acc(dy[row * lddy + c]) - dot));
    }
  }
}

// ============================================================================
// mean-error norm -- fused_ops.py:295-423 (+ dgamma, fused_ops.py:593-597)
// ============================================================================

// Vectors of V elements of type R (the residual branch may be narrower than
// the residual stream: 8-byte loads of 4 bf16 beside 16-byte loads of 4 fp32).
template <typename R, int V>
__device__ __forceinline__ VecT<R, V> ld_vec_any(const R* __restrict__ p) {
  if constexpr (sizeof(VecT<R, V>) == 16) {
    return ld_vec<R, V>(p);
  } else {
    static_assert(sizeof(VecT<R, V>) == 8, "8- or 16-byte vectors");
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return __builtin_bit_cast(VecT<R, V>, r);
  }
}
template <typename R, int V>
__device__ __forceinline__ void st_vec_any(R* __restrict__ p, const VecT<R, V>& v) {
  if constexpr (sizeof(VecT<R, V>) == 16) {
    st_vec<R, V>(p, v);
  } else {
    static_assert(sizeof(VecT<R, V>) == 8, "8- or 16-byte vectors");
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2_t*>(p) = __builtin_bit_cast(u32x2_t, v);
  }
}
template <typename R, int V, int NCH, bool FULL = false>
__device__ __forceinline__ void load_row_any(const R* __restrict__ base, int n_cols,
                                             VecT<R, V> (&r)[NCH]) {
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = ((int)threadIdx.x + 256 * k) * V;
    r[k] = ld_vec_any<R, V>(base + ((FULL || col < n_cols) ? col : 0));
  }
}

// R = void: y = norm(x). Otherwise the residual add in front of the norm is
// fused in (the block's `x = x + branch(...)` followed by norm2 / the next
// norm1, algebraic_model.py:150-151): h = x + r is rounded to T exactly as
// torch's promoted add rounds it, written once, and normalised from registers,
// so (h, y, mu) are bit-identical to the add followed by the plain norm.
template <typename T, typename W, int NCH, typename R = void, typename Y = T, bool FULL = false>
__global__ __launch_bounds__(256) void men_fwd_k(const T* __restrict__ x, const W* __restrict__ w,
                                                 Y* __restrict__ y, float* __restrict__ mu,
                                                 int64_t n_rows, int n_cols, int64_t ldx,
                                                 int64_t ldy, float eps, const void* __restrict__ rp,
                                                 T* __restrict__ h, int64_t ldr, int64_t ldh) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  constexpr bool kAdd = !std::is_void<R>::value;
  typedef std::conditional_t<kAdd, R, T> RT;
  const RT* r = reinterpret_cast<const RT*>(rp);
  __shared__ A red[2][kRowWaves];
  A wv[NCH][V];
  load_weight<T, W, NCH>(w, n_cols, wv);
  const int64_t G = gridDim.x;
  int64_t row = blockIdx.x;
  const int64_t last = n_rows - 1;
  VecT<T, V> cur[NCH], nx1[NCH];
  VecT<RT, V> rc[NCH], r1[NCH];
  load_row<T, NCH, FULL>(x + std::min(row, last) * ldx, n_cols, cur);
  if constexpr (kAdd) load_row_any<RT, V, NCH, FULL>(r + std::min(row, last) * ldr, n_cols, rc);
  load_row<T, NCH, FULL>(x + std::min(row + G, last) * ldx, n_cols, nx1);
  if constexpr (kAdd) load_row_any<RT, V, NCH, FULL>(r + std::min(row + G, last) * ldr, n_cols, r1);
  for (int par = 0; row < n_rows; row += G, par ^= 1) {
    VecT<T, V> nx2[NCH];
    VecT<RT, V> r2[NCH];
    load_row<T, NCH, FULL>(x + std::min(row + 2 * G, last) * ldx, n_cols, nx2);
    if constexpr (kAdd) {
      load_row_any<RT, V, NCH, FULL>(r + std::min(row + 2 * G, last) * ldr, n_cols, r2);
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int col = ((int)threadIdx.x + 256 * k) * V;
#pragma unroll
        for (int i = 0; i < V; ++i)
          cur[k].v[i] = from_acc<T>(to_acc(cur[k].v[i]) + to_acc(rc[k].v[i]));
        if (FULL || col < n_cols) st_vec<T, V>(h + row * ldh + col, cur[k]);
      }
    }
    A s = A(0);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const bool in = chunk_in<FULL>(k, V, n_cols);
#pragma unroll
      for (int i = 0; i < V; ++i) s += in ? fabs(to_acc(cur[k].v[i])) : A(0);  // fused_ops.py:324
    }
    s = block_sum_par(s, red, par);
    const A mean = s / A(n_cols);          // fused_ops.py:326
    const A inv = A(1) / (mean + A(eps));  // fused_ops.py:327
    if (threadIdx.x == 0) mu[row] = (float)mean;  // fused_ops.py:330 (no eps)
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int col = ((int)threadIdx.x + 256 * k) * V;
      if (FULL || col < n_cols) {
        VecT<Y, V> o;
#pragma unroll
        for (int i = 0; i < V; ++i) o.v[i] = narrow_to<Y>(to_acc(cur[k].v[i]) * inv * wv[k][i]);  // :340
        st_vec_any<Y, V>(y + row * ldy + col, o);
      }
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      cur[k] = nx1[k];
      nx1[k] = nx2[k];
      if constexpr (kAdd) {
        rc[k] = r1[k];
        r1[k] = r2[k];
      }
    }
  }
}

// Each thread owns fixed columns, so its dgamma partial over the block's rows
// needs no cross-thread reduction: it goes straight to partial[block][col].
// Each block keeps kNormPf rows in flight ahead of the one it is reducing.
constexpr int kNormPf = 2;

// R = void: the norm's backward. Otherwise the backward of the fused
// residual add + norm: x is then h = x + r, dh the gradient that reaches h
// through the residual stream, and dx = round_T(norm_bwd) + dh (the sum
// autograd forms for h, in T), written for x and, cast to R, for r (dr may
// be null).
template <typename T, typename W, int NCH, typename R = void, typename Y = T, bool FULL = false>
__global__ __launch_bounds__(256) void men_bwd_k(
    const Y* __restrict__ dy, const T* __restrict__ x, const W* __restrict__ w,
    const float* __restrict__ mu, T* __restrict__ dx, typename AccT<T>::type* __restrict__ partial,
    int64_t n_rows, int n_cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps,
    const T* __restrict__ dh, int64_t lddh, void* __restrict__ drp, int64_t lddr) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  constexpr int PF = kNormPf;
  constexpr bool kAdd = !std::is_void<R>::value;
  typedef std::conditional_t<kAdd, R, T> RT;
  RT* dr = reinterpret_cast<RT*>(drp);
  __shared__ A red[2][kRowWaves];
  A wv[NCH][V], dg[NCH][V];
  load_weight<T, W, NCH>(w, n_cols, wv);
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int i = 0; i < V; ++i) dg[k][i] = A(0);
  const A e = A(eps);
  const int64_t G = gridDim.x;
  int64_t row = blockIdx.x;
  // ring of rows row, row + G, ..., row + PF*G: slot 0 is reduced next
  VecT<Y, V> by[PF + 1][NCH];
  VecT<T, V> bx[PF + 1][NCH], bh[PF + 1][NCH];
  float bm[PF + 1];
  // Rows past the end are clamped to the last row (loaded, never used):
  // a conditional load would make the compiler wait for it on the spot.
  const int64_t last = n_rows - 1;
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int64_t r = std::min(row + j * G, last);
    load_row_any<Y, V, NCH, FULL>(dy + r * lddy, n_cols, by[j]);
    load_row<T, NCH, FULL>(x + r * ldx, n_cols, bx[j]);
    if constexpr (kAdd) load_row<T, NCH, FULL>(dh + r * lddh, n_cols, bh[j]);
    bm[j] = mu[r];  // the row statistic travels with its row
  }
  for (int par = 0; row < n_rows; row += G, par ^= 1) {
    {
      const int64_t r = std::min(row + PF * G, last);
      load_row_any<Y, V, NCH, FULL>(dy + r * lddy, n_cols, by[PF]);
      load_row<T, NCH, FULL>(x + r * ldx, n_cols, bx[PF]);
      if constexpr (kAdd) load_row<T, NCH, FULL>(dh + r * lddh, n_cols, bh[PF]);
      bm[PF] = mu[r];
    }
    const A inv = A(1) / ((A)bm[0] + e);  // fused_ops.py:389-390
    A cs = A(0);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const bool in = chunk_in<FULL>(k, V, n_cols);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A p = to_acc(bx[0][k].v[i]) * inv * wv[k][i];
        cs = in ? men_fma(to_acc(by[0][k].v[i]), p, cs) : cs;  // fused_ops.py:404-405
      }
    }
    cs = block_sum_par(cs, red, par);
    const A corr = cs / A(n_cols);  // fused_ops.py:408
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int col = ((int)threadIdx.x + 256 * k) * V;
      const bool in = FULL || col < n_cols;
      VecT<T, V> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const A yy = to_acc(by[0][k].v[i]);
        const A xx = to_acc(bx[0][k].v[i]);
        o.v[i] = narrow_to<T>(men_dx(yy, xx, wv[k][i], inv, corr));  // fused_ops.py:418-421
        if constexpr (kAdd) o.v[i] = from_acc<T>(to_acc(o.v[i]) + to_acc(bh[0][k].v[i]));
        dg[k][i] = in ? men_fma(yy, xx * inv, dg[k][i]) : dg[k][i];  // fused_ops.py:595-597
      }
      if (in) st_vec<T, V>(dx + row * lddx + col, o);
      if constexpr (kAdd) {
        if (in && dr != nullptr) {
          VecT<RT, V> od;
#pragma unroll
          for (int i = 0; i < V; ++i) od.v[i] = narrow_to<RT>(to_acc(o.v[i]));
          st_vec_any<RT, V>(dr + row * lddr + col, od);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      bm[j] = bm[j + 1];
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        by[j][k] = by[j + 1][k];
        bx[j][k] = bx[j + 1][k];
        if constexpr (kAdd) bh[j][k] = bh[j + 1][k];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = ((int)threadIdx.x + 256 * k) * V;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (FULL || col + i < n_cols) partial[(int64_t)blockIdx.x * n_cols + col + i] = dg[k][i];
  }
}

// h = x + r (R non-void) is formed in the first pass, written, and formed
// again from x and r in the second (the same rounding, so the same value).
template <typename T, typename R = void, typename Y = T>
__global__ __launch_bounds__(256) void men_fwd_mp_k(const T* __restrict__ x, const void* __restrict__ wp,
                                                    int w_is_f32, Y* __restrict__ y,
                                                    float* __restrict__ mu, int64_t n_rows,
                                                    int n_cols, int64_t ldx, int64_t ldy,
                                                    float eps, const void* __restrict__ rp,
                                                    T* __restrict__ h, int64_t ldr, int64_t ldh) {
  typedef typename AccT<T>::type A;
  constexpr bool kAdd = !std::is_void<R>::value;
  typedef std::conditional_t<kAdd, R, T> RT;
  const RT* r = reinterpret_cast<const RT*>(rp);
  __shared__ A sh[kRowWaves];
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    auto xin = [&](int c) -> T {
      if constexpr (kAdd) return from_acc<T>(to_acc(x[row * ldx + c]) + to_acc(r[row * ldr + c]));
      else return x[row * ldx + c];
    };
    A s = A(0);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const T xv = xin(c);
      if constexpr (kAdd) h[row * ldh + c] = xv;
      s += fabs(to_acc(xv));
    }
    s = block_sum(s, sh);
    const A mean = s / A(n_cols);
    const A inv = A(1) / (mean + A(eps));
    if (threadIdx.x == 0) mu[row] = (float)mean;
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
      y[row * ldy + c] = narrow_to<Y>(to_acc(xin(c)) * inv * wv);
    }
  }
}

template <typename T, typename R = void, typename Y = T>
__global__ __launch_bounds__(256) void men_bwd_mp_k(
    const Y* __restrict__ dy, const T* __restrict__ x, const void* __restrict__ wp, int w_is_f32,
    const float* __restrict__ mu, T* __restrict__ dx, typename AccT<T>::type* __restrict__ partial,
    int64_t n_rows, int n_cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps,
    const T* __restrict__ dh, int64_t lddh, void* __restrict__ drp, int64_t lddr) {
  typedef typename AccT<T>::type A;
  constexpr bool kAdd = !std::is_void<R>::value;
  typedef std::conditional_t<kAdd, R, T> RT;
  RT* dr = reinterpret_cast<RT*>(drp);
  __shared__ A sh[kRowWaves];
  A* part = partial + (int64_t)blockIdx.x * n_cols;  // owned by this block
  for (int c = threadIdx.x; c < n_cols; c += blockDim.x) part[c] = A(0);
  const A e = A(eps);
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const A inv = A(1) / ((A)mu[row] + e);
    A cs = A(0);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
      cs = men_fma(to_acc(dy[row * lddy + c]), to_acc(x[row * ldx + c]) * inv * wv, cs);
    }
    cs = block_sum(cs, sh);
    const A corr = cs / A(n_cols);
    for (int c = threadIdx.x; c < n_cols; c += blockDim.x) {
      const A wv = w_is_f32 ? (A)((const float*)wp)[c] : to_acc(((const T*)wp)[c]);
      const A yy = to_acc(dy[row * lddy + c]);
      const A xx = to_acc(x[row * ldx + c]);
      T g = narrow_to<T>(men_dx(yy, xx, wv, inv, corr));
      if constexpr (kAdd) {
        g = from_acc<T>(to_acc(g) + to_acc(dh[row * lddh + c]));
        if (dr != nullptr) dr[row * lddr + c] = narrow_to<RT>(to_acc(g));
      }
      dx[row * lddx + c] = g;
      part[c] = men_fma(yy, xx * inv, part[c]);  // same thread owns column c throughout
    }
  }
}

// dw[c] = sum_g partial[g][c] in a fixed order. A block owns 16 columns and
// 64 row groups (4 per wave, 16 waves): row group rg adds rows rg, rg + 64, ...
// in two interleaved accumulators, then the 64 group sums are added in group
// order. 16 columns per block give cols / 16 blocks (256 at 4096 columns), so
// the reduction spreads over the whole chip.
// 16 fp32 columns are half a 128-byte line: the two blocks that share a line
// are blocks b and b + 8, which the dispatcher places on the same XCD (blocks
// go round-robin over the 8 XCDs), so the line crosses HBM once for both
// (adjacent blocks, on two XCDs with separate L2s, fetched every line twice).
template <typename A>
__global__ __launch_bounds__(1024) void colsum_k(const A* __restrict__ partial, int G, int n_cols,
                                                 A* __restrict__ out) {
  __shared__ A red[64][17];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, rg = wave * 4 + (lane >> 4);
  const int b = blockIdx.x, nb16 = (int)gridDim.x & ~15;
  const int cg = b < nb16 ? (((b >> 4) * 8 + (b & 7)) * 2 + ((b >> 3) & 1)) : b;
  const int col = cg * 16 + c;
  A s0 = A(0), s1 = A(0);
  if (col < n_cols) {
    int g = rg;
    for (; g + 64 < G; g += 128) {
      s0 += partial[(int64_t)g * n_cols + col];
      s1 += partial[(int64_t)(g + 64) * n_cols + col];
    }
    for (; g < G; g += 64) s0 += partial[(int64_t)g * n_cols + col];
  }
  red[rg][c] = s0 + s1;
  __syncthreads();
  if (threadIdx.x < 16 && cg * 16 + (int)threadIdx.x < n_cols) {
    A t = A(0);
#pragma unroll 8
    for (int i = 0; i < 64; ++i) t += red[i][threadIdx.x];
    out[cg * 16 + threadIdx.x] = t;
  }
}

template <typename A> __global__ void fill_zero_k(A* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = A(0);
}

// ============================================================================
// Host launchers
// ============================================================================

// Persistent row grids: up to `per_cu` 256-thread blocks per compute unit,
// and at least 4 rows per block so the two-row prefetch (which clamps past
// the last row) wastes little.
constexpr int kRowBlocksPerCU = 8;
static inline int64_t row_grid(int64_t rows, int per_cu) {
  const int64_t cap = std::min<int64_t>((int64_t)per_cu * num_cus(), (rows + 3) / 4);
  return std::max<int64_t>(1, std::min<int64_t>(rows, cap));
}

// grid of the one-block-per-row kernels, which walk rows with a grid stride
// (so row counts past 2^31 stay covered)
static inline unsigned mp_grid(int64_t rows) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t)1 << 30));
}

static inline int pick_nch(int64_t n_cols, int per) {
  const int64_t need = (n_cols + per - 1) / per;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  if (need <= 16) return 16;
  return 0;
}

// Few enough rows for the one-wave-per-row kernels: every row's wave resident
// at once (at most 16 per CU). They take rows of up to 8 chunks per lane (512
// bf16 / 256 fp32 values per chunk round); wider rows would hold more
// registers than leave room for the waves.
static inline bool wave_rows(int64_t rows) { return rows <= (int64_t)16 * num_cus(); }
#define KAT_NCH_SWITCH8(nch, ...)                         \
  switch (nch) {                                          \
    case 1: { constexpr int N = 1; __VA_ARGS__; } break;  \
    case 2: { constexpr int N = 2; __VA_ARGS__; } break;  \
    case 4: { constexpr int N = 4; __VA_ARGS__; } break;  \
    default: { constexpr int N = 8; __VA_ARGS__; } break; \
  }

// The predicate-free (FULL) norm kernels exist for 2 and 4 chunk rounds: rows
// of 4096 / 8192 bf16 or 2048 / 4096 fp32 values, the benchmark's and model
// widths (measured 4% faster backward at 16384 x 4096); at 8 rounds the 16-bit
// residual-add backward would spill.
constexpr bool kat_full_nch(int n) { return n == 2 || n == 4; }
static inline bool kat_full_variant(int n, bool full) { return full && kat_full_nch(n); }

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
    hipLaunchKernelGGL((swiglu_fwd_scalar_k<T>), scalar_grid(rows, cols), dim3(kEwThreads), 0, st, g,
                       v, o, rows, cols, ldg, ldv, ldo);
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
    hipLaunchKernelGGL((swiglu_bwd_scalar_k<T>), scalar_grid(rows, cols), dim3(kEwThreads), 0, st, dy,
                       g, v, dg, dv, rows, cols, lddy, ldg, ldv, lddg, lddv);
  }
  return check_launch("kat_rswiglu_bwd");
}

template <typename T>
static int rsoftmax_fwd_t(const T* x, T* p, int64_t rows, int64_t cols, int64_t ldx, int64_t ldp,
                          float eps, hipStream_t st) {
  constexpr int V = Raw<T>::V;
  const bool vec = cols % V == 0 && ldx % V == 0 && ldp % V == 0 && aligned16(x) && aligned16(p);
  const int nch = vec ? pick_nch(cols, 256 * V) : 0;
  const int nchw = vec && wave_rows(rows) ? pick_nch(cols, 64 * V) : 0;
  if (nchw && nchw <= 8) {
    const unsigned blocks = (unsigned)((rows + kRowWaves - 1) / kRowWaves);
    KAT_NCH_SWITCH8(nchw, hipLaunchKernelGGL((rsoftmax_fwd_w_k<T, N>), dim3(blocks), dim3(256), 0, st,
                                            x, p, rows, (int)cols, ldx, ldp, eps));
  } else if (nch) {
    const int64_t blocks = row_grid(rows, kRowBlocksPerCU);
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((rsoftmax_fwd_k<T, N>), dim3((unsigned)blocks),
                                           dim3(256), 0, st, x, p, rows, (int)cols, ldx, ldp, eps));
  } else {
    hipLaunchKernelGGL((rsoftmax_fwd_mp_k<T>), dim3(mp_grid(rows)), dim3(256), 0, st, x, p, rows,
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
  const int nch = vec ? pick_nch(cols, 256 * V) : 0;
  const int nchw = vec && wave_rows(rows) ? pick_nch(cols, 64 * V) : 0;
  if (nchw && nchw <= 8) {
    const unsigned blocks = (unsigned)((rows + kRowWaves - 1) / kRowWaves);
    KAT_NCH_SWITCH8(nchw, hipLaunchKernelGGL((rsoftmax_bwd_w_k<T, N>), dim3(blocks), dim3(256), 0, st,
                                            dy, x, p, dx, rows, (int)cols, lddy, ldx, ldp, lddx,
                                            eps));
  } else if (nch) {
    const int64_t blocks = row_grid(rows, kRowBlocksPerCU);
    KAT_NCH_SWITCH(nch, hipLaunchKernelGGL((rsoftmax_bwd_k<T, N>), dim3((unsigned)blocks),
                                           dim3(256), 0, st, dy, x, p, dx, rows, (int)cols, lddy,
                                           ldx, ldp, lddx, eps));
  } else {
    hipLaunchKernelGGL((rsoftmax_bwd_mp_k<T>), dim3(mp_grid(rows)), dim3(256), 0, st, dy, x, p,
                       dx, rows, (int)cols, lddy, ldx, ldp, lddx, eps);
  }
  return check_launch("kat_rsoftmax_bwd");
}

template <typename T, typename W, typename R = void, typename Y = T>
static int men_fwd_t(const T* x, const W* w, Y* y, float* mu, int64_t rows, int64_t cols,
                     int64_t ldx, int64_t ldy, float eps, hipStream_t st, const R* r = nullptr,
                     T* h = nullptr, int64_t ldr = 0, int64_t ldh = 0) {
  constexpr int V = Raw<T>::V;
  constexpr bool kAdd = !std::is_void<R>::value;
  bool vec = cols % V == 0 && ldx % V == 0 && ldy % V == 0 && aligned16(x) &&
             reinterpret_cast<uintptr_t>(y) % (V * sizeof(Y)) == 0 && aligned16(w);
  if constexpr (kAdd)
    vec = vec && ldr % V == 0 && ldh % V == 0 && aligned16(h) &&
          reinterpret_cast<uintptr_t>(r) % (V * sizeof(R)) == 0;
  const int nch = vec ? pick_nch(cols, 256 * V) : 0;
  if (nch) {
    const int64_t blocks = row_grid(rows, kRowBlocksPerCU);
    const bool full = cols == (int64_t)nch * 256 * V;
    KAT_NCH_SWITCH(nch, {
      if (kat_full_variant(N, full))
        hipLaunchKernelGGL((men_fwd_k<T, W, N, R, Y, kat_full_nch(N)>), dim3((unsigned)blocks),
                           dim3(256), 0, st, x, w, y, mu, rows, (int)cols, ldx, ldy, eps,
                           (const void*)r, h, ldr, ldh);
      else
        hipLaunchKernelGGL((men_fwd_k<T, W, N, R, Y>), dim3((unsigned)blocks), dim3(256), 0, st, x,
                           w, y, mu, rows, (int)cols, ldx, ldy, eps, (const void*)r, h, ldr, ldh);
    });
  } else {
    hipLaunchKernelGGL((men_fwd_mp_k<T, R, Y>), dim3(mp_grid(rows)), dim3(256), 0, st, x,
                       (const void*)w, (int)std::is_same<W, float>::value, y, mu, rows, (int)cols,
                       ldx, ldy, eps, (const void*)r, h, ldr, ldh);
  }
  return check_launch(kAdd ? "kat_add_men_fwd" : "kat_men_fwd");
}

// dgamma partials cost G x cols x 4 bytes of extra traffic (written here,
// read by colsum_k): two blocks per CU.
static int men_bwd_grid(int64_t rows, bool resident) {
  (void)resident;
  return (int)row_grid(rows, 2);
}

template <typename T, typename W, typename R = void, typename Y = T>
static int men_bwd_t(const Y* dy, const T* x, const W* w, const float* mu, T* dx,
                     typename AccT<T>::type* dw, void* ws, size_t ws_bytes, int64_t rows,
                     int64_t cols, int64_t lddy, int64_t ldx, int64_t lddx, float eps,
                     hipStream_t st, const T* dh = nullptr, int64_t lddh = 0, R* dr = nullptr,
                     int64_t lddr = 0) {
  typedef typename AccT<T>::type A;
  constexpr int V = Raw<T>::V;
  constexpr bool kAdd = !std::is_void<R>::value;
  const char* nm = kAdd ? "kat_add_men_bwd" : "kat_men_bwd";
  bool vec = cols % V == 0 && lddy % V == 0 && ldx % V == 0 && lddx % V == 0 &&
             reinterpret_cast<uintptr_t>(dy) % (V * sizeof(Y)) == 0 && aligned16(x) &&
             aligned16(dx) && aligned16(w);
  if constexpr (kAdd)
    vec = vec && lddh % V == 0 && aligned16(dh) &&
          (dr == nullptr || (lddr % V == 0 && reinterpret_cast<uintptr_t>(dr) % (V * sizeof(R)) == 0));
  const int nch = vec ? pick_nch(cols, 256 * V) : 0;
  const int G = men_bwd_grid(rows, nch != 0);
  const size_t need = (size_t)G * (size_t)cols * sizeof(A);
  if (ws_bytes < need || (need && ws == nullptr))
    return fail(KAT_EINVAL, "%s: workspace %zu bytes < required %zu", nm, ws_bytes, need);
  A* partial = reinterpret_cast<A*>(ws);
  if (nch) {
    const bool full = cols == (int64_t)nch * 256 * V;
    KAT_NCH_SWITCH(nch, {
      if (kat_full_variant(N, full))
        hipLaunchKernelGGL((men_bwd_k<T, W, N, R, Y, kat_full_nch(N)>), dim3(G), dim3(256), 0, st,
                           dy, x, w, mu, dx, partial, rows, (int)cols, lddy, ldx, lddx, eps, dh,
                           lddh, (void*)dr, lddr);
      else
        hipLaunchKernelGGL((men_bwd_k<T, W, N, R, Y>), dim3(G), dim3(256), 0, st, dy, x, w, mu, dx,
                           partial, rows, (int)cols, lddy, ldx, lddx, eps, dh, lddh, (void*)dr,
                           lddr);
    });
  } else {
    hipLaunchKernelGGL((men_bwd_mp_k<T, R, Y>), dim3(G), dim3(256), 0, st, dy, x, (const void*)w,
                       (int)std::is_same<W, float>::value, mu, dx, partial, rows, (int)cols, lddy,
                       ldx, lddx, eps, dh, lddh, (void*)dr, lddr);
  }
  int rc = check_launch(nm);
  if (rc) return rc;
  hipLaunchKernelGGL((colsum_k<A>), dim3((unsigned)((cols + 15) / 16)), dim3(1024), 0, st,
                     partial, G, (int)cols, dw);
  return check_launch(kAdd ? "kat_add_men_bwd (dw reduction)" : "kat_men_bwd (dw reduction)");
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

// Residual add fused with the norm. The residual branch r (and its gradient
// dr) has the stream's dtype, or bf16 / fp16 beside an fp32 stream (the
// branch output of an autocast matmul added to the fp32 residual); so has the
// normalised output y (and its gradient dy): an autocast matmul reads it in
// its own dtype, so y is rounded once, as the cast would.
#define KAT_NARROW_SWITCH(code, U, dtype, ...)                                          \
  if ((code) == (dtype)) { typedef T U; __VA_ARGS__; }                                 \
  if constexpr (std::is_same<T, float>::value) {                                        \
    if ((code) == KAT_BF16) { typedef bf16 U; __VA_ARGS__; }                            \
    if ((code) == KAT_F16) { typedef f16 U; __VA_ARGS__; }                              \
  }

template <typename T, typename W>
static int add_men_fwd_d(const char* nm, int dtype, int dtype_r, int dtype_y, const void* x,
                         const void* r, const void* w, void* h, void* y, float* mu, int64_t rows,
                         int64_t cols, int64_t ldx, int64_t ldr, int64_t ldh, int64_t ldy,
                         float eps, hipStream_t st) {
  KAT_NARROW_SWITCH(dtype_r, R, dtype,
    KAT_NARROW_SWITCH(dtype_y, Y, dtype,
      return (men_fwd_t<T, W, R, Y>((const T*)x, (const W*)w, (Y*)y, mu, rows, cols, ldx, ldy, eps,
                                    st, (const R*)r, (T*)h, ldr, ldh))))
  return fail(KAT_EUNSUPPORTED, "%s: residual dtype %d / output dtype %d with stream dtype %d", nm,
              dtype_r, dtype_y, dtype);
}

template <typename T, typename W>
static int add_men_bwd_d(const char* nm, int dtype, int dtype_r, int dtype_y, const void* dy,
                         const void* dh, const void* h, const void* w, const float* mu, void* dx,
                         void* dr, void* dw, void* ws, size_t ws_bytes, int64_t rows, int64_t cols,
                         int64_t lddy, int64_t lddh, int64_t ldh, int64_t lddx, int64_t lddr,
                         float eps, hipStream_t st) {
  typedef typename AccT<T>::type A;
  KAT_NARROW_SWITCH(dtype_r, R, dtype,
    KAT_NARROW_SWITCH(dtype_y, Y, dtype,
      return (men_bwd_t<T, W, R, Y>((const Y*)dy, (const T*)h, (const W*)w, mu, (T*)dx, (A*)dw, ws,
                                    ws_bytes, rows, cols, lddy, ldh, lddx, eps, st, (const T*)dh,
                                    lddh, (R*)dr, lddr))))
  return fail(KAT_EUNSUPPORTED, "%s: residual dtype %d / output dtype %d with stream dtype %d", nm,
              dtype_r, dtype_y, dtype);
}

extern "C" int kat_add_men_fwd(const void* x, const void* r, const void* w, void* h, void* y,
                               float* mu, int64_t n_rows, int64_t n_cols, int64_t ld_x,
                               int64_t ld_r, int64_t ld_h, int64_t ld_y, float eps, int dtype,
                               int dtype_r, int dtype_y, int dtype_w, void* stream) {
  const char* nm = "kat_add_men_fwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_rows == 0 || n_cols == 0) return KAT_OK;
  if (!x || !r || !w || !h || !y || !mu) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_x, ld_r, ld_h, ld_y})) return rc;
  const hipStream_t st = as_stream(stream);
  if (dtype_w == dtype) {
    KAT_DISPATCH_T(dtype, nm,
                   (add_men_fwd_d<T, T>(nm, dtype, dtype_r, dtype_y, x, r, w, h, y, mu, n_rows,
                                        n_cols, ld_x, ld_r, ld_h, ld_y, eps, st)));
  }
  if (dtype_w == KAT_F32 && dtype != KAT_F64) {
    KAT_DISPATCH_T(dtype, nm,
                   (add_men_fwd_d<T, float>(nm, dtype, dtype_r, dtype_y, x, r, w, h, y, mu, n_rows,
                                            n_cols, ld_x, ld_r, ld_h, ld_y, eps, st)));
  }
  return fail(KAT_EUNSUPPORTED, "%s: weight dtype %d with input dtype %d", nm, dtype_w, dtype);
}

extern "C" int kat_add_men_bwd(const void* dy, const void* dh, const void* h, const void* w,
                               const float* mu, void* dx, void* dr, void* dw, void* workspace,
                               size_t workspace_bytes, int64_t n_rows, int64_t n_cols,
                               int64_t ld_dy, int64_t ld_dh, int64_t ld_h, int64_t ld_dx,
                               int64_t ld_dr, float eps, int dtype, int dtype_r, int dtype_y,
                               int dtype_w, void* stream) {
  const char* nm = "kat_add_men_bwd";
  if (int rc = check_rows(nm, n_rows, n_cols)) return rc;
  if (n_cols == 0) return KAT_OK;
  if (n_rows == 0)  // dw = 0, like kat_men_bwd
    return kat_men_bwd(dy, h, w, mu, dx, dw, workspace, workspace_bytes, 0, n_cols, n_cols,
                       n_cols, n_cols, eps, dtype, dtype_w, stream);
  if (!dy || !dh || !h || !w || !mu || !dx || !dw) return fail(KAT_EINVAL, "%s: null pointer", nm);
  if (int rc = check_ld(nm, n_cols, {ld_dy, ld_dh, ld_h, ld_dx})) return rc;
  if (dr != nullptr)
    if (int rc = check_ld(nm, n_cols, {ld_dr})) return rc;
  const hipStream_t st = as_stream(stream);
  if (dtype_w == dtype) {
    KAT_DISPATCH_T(dtype, nm,
                   (add_men_bwd_d<T, T>(nm, dtype, dtype_r, dtype_y, dy, dh, h, w, mu, dx, dr, dw,
                                        workspace, workspace_bytes, n_rows, n_cols, ld_dy, ld_dh,
                                        ld_h, ld_dx, ld_dr, eps, st)));
  }
  if (dtype_w == KAT_F32 && dtype != KAT_F64) {
    KAT_DISPATCH_T(dtype, nm,
                   (add_men_bwd_d<T, float>(nm, dtype, dtype_r, dtype_y, dy, dh, h, w, mu, dx, dr, dw,
                                            workspace, workspace_bytes, n_rows, n_cols, ld_dy,
                                            ld_dh, ld_h, ld_dx, ld_dr, eps, st)));
  }
  return fail(KAT_EUNSUPPORTED, "%s: weight dtype %d with input dtype %d", nm, dtype_w, dtype);
}
