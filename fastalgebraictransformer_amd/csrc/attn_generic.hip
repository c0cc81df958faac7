// Rational attention on gfx950 -- tiled kernels on the vector ALUs.
//
// These kernels compute in fp32 FMA (fp64 for fp64 tensors) on the vector
// ALUs, with square query/key tiles staged through LDS. They serve fp32 and
// fp64 inputs, head dims the MFMA kernels do not cover (any D <= 1024), and
// are the independent on-GPU cross-check of the bf16 MFMA kernels. The tile
// edge TB is 32 rows while four TB x (D + 1) tiles of the accumulation type
// fit the LDS (fp32 up to D = 256), and halves for wider rows or fp64.
//
// Math (reference forward.py:110-159, backward.py:116-154, 222-260):
//   s_ij = (q_i . k_j) * scale - slope_h * |i - j|,  j <= i (causal), every j
//   (causal == 0); keys the padding mask drops are skipped
//   f_ij = sigma(s_ij)^4, L_i = sum_j f_ij (stored without eps, fp32)
//   o_i  = sum_j f_ij v_j / (L_i + eps)
//   p = f / (L + eps), g = 2 / ((|s|+1)^2 (sigma + eps)), dS = p g (dO_i.v_j - Delta_i)
//   dq = scale * sum_j dS k_j,  dk = scale * sum_i dS q_i,  dv = sum_i p dO_i
// In causal mode keys j > i are never visited, exactly as the reference
// kernels' loops. The reference computes in fp32 for every input dtype
// (forward.py:103 `.to(tl.float32)`); fp64 tensors here keep fp64 arithmetic,
// as the row ops do, so that fp64 gradient checks hold.

#include <algorithm>

#include "kat_common.h"
#include "kat_internal.h"
#include "attn_common.h"

namespace kat {

// Tile edge for rows of DMAX elements of BYTES each: 32, halved until the four
// row tiles and the two score tiles fit ~150 KB of LDS.
template <int BYTES, int DMAX> constexpr int gen_tb() {
  int tb = 32;
  while (tb > 4 && (4 * tb * (DMAX + 1) + 2 * tb * (tb + 1)) * BYTES > 150 * 1024) tb /= 2;
  return tb;
}

template <typename A, int DMAX, int TB> struct GenericTiles {
  A a[TB][DMAX + 1];  // Q (fwd, dq) or K (dkv)
  A b[TB][DMAX + 1];  // K (fwd, dq) or V (dkv)
  A c[TB][DMAX + 1];  // V (fwd), dO (dq), Q (dkv)
  A d[TB][DMAX + 1];  // unused (fwd), V (dq), dO (dkv)
  A p[TB][TB + 1];    // f / p tile
  A s[TB][TB + 1];    // dS tile
  A r0[TB], r1[TB];   // per-row L / Delta
};

// Thread layout of a 256-thread block over TB x TB tiles: output rows are
// worked by TPR = 256 / TB consecutive threads (row tid / TPR, columns
// cl + TPR m); scores are spread one per thread (row idx / TB, column
// idx % TB for idx = tid + 256 m), each a sequential dot product over d.
template <typename T, typename A, int DMAX, int TB>
__device__ __forceinline__ void load_tile(A (*dst)[DMAX + 1], const T* __restrict__ src, int64_t st,
                                          int row0, int n_rows, int D) {
  for (int idx = threadIdx.x; idx < TB * DMAX; idx += blockDim.x) {
    const int r = idx / DMAX, d = idx - r * DMAX;
    A val = A(0);
    if (d < D && row0 + r < n_rows) val = (A)src[(int64_t)(row0 + r) * st + d];
    dst[r][d] = val;
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_fwd_generic_k(AttnArgs a) {
  typedef typename AccT<T>::type A;
  constexpr int TB = gen_tb<sizeof(A), DMAX>(), TPR = 256 / TB, NO = DMAX / TPR;
  __shared__ GenericTiles<A, DMAX, TB> sm;
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int q0 = blockIdx.x * TB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const A slope = a.slopes[h], scale = a.scale;
  const int tid = threadIdx.x, r = tid / TPR, cl = tid % TPR;
  const int i = q0 + r;

  load_tile<T, A, DMAX, TB>(sm.a, q, a.sq[2], q0, T_, D);
  A acc[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) acc[m] = A(0);
  A l = A(0);
  const bool causal = a.causal != 0;
  const int kend = causal ? std::min(q0 + TB, T_) : T_;  // causal: keys < q0 + TB
  for (int k0 = 0; k0 < kend; k0 += TB) {
    __syncthreads();
    load_tile<T, A, DMAX, TB>(sm.b, k, a.sk[2], k0, T_, D);
    load_tile<T, A, DMAX, TB>(sm.c, v, a.sv[2], k0, T_, D);
    __syncthreads();
    for (int idx = tid; idx < TB * TB; idx += 256) {
      const int sr = idx / TB, c = idx % TB, si = q0 + sr, j = k0 + c;
      A dot = A(0);
      for (int d = 0; d < D; ++d) dot = fma(sm.a[sr][d], sm.b[c][d], dot);
      const A s = dot * scale - slope * (A)abs(si - j);  // forward.py:129-133
      const A sg = rsig(s);                              // forward.py:137-140
      const A s2 = sg * sg;
      const bool vis = (causal ? j <= si : j < T_) && si < T_ && key_ok(a, b, j);
      sm.p[sr][c] = vis ? s2 * s2 : A(0);
    }
    __syncthreads();
    for (int c = 0; c < TB; ++c) {
      const A f = sm.p[r][c];
      l += f;  // forward.py:142
#pragma unroll
      for (int m = 0; m < NO; ++m) acc[m] = fma(f, sm.c[c][cl + TPR * m], acc[m]);  // :147
    }
  }
  if (i < T_) {
    const A inv = A(1) / (l + (A)a.eps);  // forward.py:150
    T* o = (T*)a.o + b * a.so[0] + h * a.so[1] + (int64_t)i * a.so[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + TPR * m;
      if (d < D) o[d] = (T)(acc[m] * inv);
    }
    if (cl == 0) a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)i * a.sl[2]] = (float)l;  // :159
  }
}

// Delta_i = <dO_i, O_i> (backward.py:117) and cinv_i = 1 / (16 (L_i + eps)),
// in the accumulation type. 16 lanes per row, 16-byte loads (VEC16) or one
// wave per row, scalar loads.
template <typename T, bool VEC16>
__global__ __launch_bounds__(256) void attn_delta_k(AttnArgs a, typename AccT<T>::type* __restrict__ delta,
                                                    typename AccT<T>::type* __restrict__ cinv) {
  typedef typename AccT<T>::type A;
  constexpr int LPR = VEC16 ? 16 : 64;  // lanes per row
  constexpr int V = VEC16 ? 16 / (int)sizeof(T) : 1;
  const int sub = threadIdx.x % LPR;
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / LPR;
  const int64_t nrows = (int64_t)a.B * a.H * a.T;
  const bool live = row < nrows;
  const int64_t rr = live ? row : 0;
  const int i = (int)(rr % a.T);
  const int64_t bh = rr / a.T;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const T* o = (const T*)a.o + b * a.so[0] + h * a.so[1] + (int64_t)i * a.so[2];
  const T* dO = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1] + (int64_t)i * a.sdo[2];
  A s = A(0);
  if (live) {
    for (int d = sub * V; d < a.D; d += LPR * V) {
      A ov[V], gv[V];
      load_acc<T, V>(o + d, ov);
      load_acc<T, V>(dO + d, gv);
#pragma unroll
      for (int e = 0; e < V; ++e) s = fma(gv[e], ov[e], s);
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (live && sub == 0) {
    delta[row] = s;
    const A l = a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)i * a.sl[2]];
    cinv[row] = A(1) / (A(16) * (l + (A)a.eps));
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_bwd_dq_generic_k(AttnArgs a,
                                                             const typename AccT<T>::type* __restrict__ delta) {
  typedef typename AccT<T>::type A;
  constexpr int TB = gen_tb<sizeof(A), DMAX>(), TPR = 256 / TB, NO = DMAX / TPR;
  __shared__ GenericTiles<A, DMAX, TB> sm;
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int q0 = blockIdx.x * TB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* dO = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const A slope = a.slopes[h], scale = a.scale, eps = a.eps;
  const int tid = threadIdx.x, r = tid / TPR, cl = tid % TPR;
  const int i = q0 + r;

  load_tile<T, A, DMAX, TB>(sm.a, q, a.sq[2], q0, T_, D);
  load_tile<T, A, DMAX, TB>(sm.c, dO, a.sdo[2], q0, T_, D);
  if (tid < TB) {
    const int ii = q0 + tid;
    sm.r0[tid] = ii < T_ ? (A)a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)ii * a.sl[2]] : A(0);
    sm.r1[tid] = ii < T_ ? delta[((int64_t)bh) * T_ + ii] : A(0);
  }
  A acc[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) acc[m] = A(0);
  const bool causal = a.causal != 0;
  const int kend = causal ? std::min(q0 + TB, T_) : T_;
  for (int k0 = 0; k0 < kend; k0 += TB) {
    __syncthreads();
    load_tile<T, A, DMAX, TB>(sm.b, k, a.sk[2], k0, T_, D);
    load_tile<T, A, DMAX, TB>(sm.d, v, a.sv[2], k0, T_, D);
    __syncthreads();
    for (int idx = tid; idx < TB * TB; idx += 256) {
      const int sr = idx / TB, c = idx % TB, si = q0 + sr, j = k0 + c;
      A dot = A(0), dp = A(0);
      for (int d = 0; d < D; ++d) {
        dot = fma(sm.a[sr][d], sm.b[c][d], dot);
        dp = fma(sm.c[sr][d], sm.d[c][d], dp);
      }
      // backward.py:133-151
      const A s = dot * scale - slope * (A)abs(si - j);
      const A den = fabs(s) + A(1);
      const A sg = A(0.5) * (s / den + A(1));
      const A s2 = sg * sg;
      const A p = s2 * s2 / (sm.r0[sr] + eps);
      const A g = A(2) / (den * den * (sg + eps));
      const bool vis = (causal ? j <= si : j < T_) && si < T_ && key_ok(a, b, j);
      sm.s[sr][c] = vis ? p * g * (dp - sm.r1[sr]) : A(0);
    }
    __syncthreads();
    for (int c = 0; c < TB; ++c) {
      const A ds = sm.s[r][c];
#pragma unroll
      for (int m = 0; m < NO; ++m) acc[m] = fma(ds, sm.b[c][cl + TPR * m], acc[m]);  // :154
    }
  }
  if (i < T_) {
    T* dq = (T*)a.dq + b * a.sdq[0] + h * a.sdq[1] + (int64_t)i * a.sdq[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + TPR * m;
      if (d < D) dq[d] = (T)(acc[m] * scale);
    }
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_bwd_dkv_generic_k(AttnArgs a,
                                                              const typename AccT<T>::type* __restrict__ delta) {
  typedef typename AccT<T>::type A;
  constexpr int TB = gen_tb<sizeof(A), DMAX>(), TPR = 256 / TB, NO = DMAX / TPR;
  __shared__ GenericTiles<A, DMAX, TB> sm;
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int k0 = blockIdx.x * TB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* dO = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const A slope = a.slopes[h], scale = a.scale, eps = a.eps;
  const int tid = threadIdx.x, r = tid / TPR, cl = tid % TPR;
  const int j = k0 + r;  // this thread's key row

  load_tile<T, A, DMAX, TB>(sm.a, k, a.sk[2], k0, T_, D);
  load_tile<T, A, DMAX, TB>(sm.b, v, a.sv[2], k0, T_, D);
  A dk[NO], dv[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) dk[m] = dv[m] = A(0);
  const bool causal = a.causal != 0;
  for (int q0 = causal ? k0 : 0; q0 < T_; q0 += TB) {  // causal: queries >= k0
    __syncthreads();
    load_tile<T, A, DMAX, TB>(sm.c, q, a.sq[2], q0, T_, D);
    load_tile<T, A, DMAX, TB>(sm.d, dO, a.sdo[2], q0, T_, D);
    if (tid < TB) {
      const int ii = q0 + tid;
      sm.r0[tid] = ii < T_ ? (A)a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)ii * a.sl[2]] : A(0);
      sm.r1[tid] = ii < T_ ? delta[((int64_t)bh) * T_ + ii] : A(0);
    }
    __syncthreads();
    for (int idx = tid; idx < TB * TB; idx += 256) {
      const int sr = idx / TB, c = idx % TB, sj = k0 + sr, i = q0 + c;
      A dot = A(0), dp = A(0);
      for (int d = 0; d < D; ++d) {
        dot = fma(sm.c[c][d], sm.a[sr][d], dot);
        dp = fma(sm.d[c][d], sm.b[sr][d], dp);
      }
      // backward.py:233-254
      const A s = dot * scale - slope * (A)abs(i - sj);
      const A den = fabs(s) + A(1);
      const A sg = A(0.5) * (s / den + A(1));
      const A s2 = sg * sg;
      const A p = s2 * s2 / (sm.r0[c] + eps);
      const A g = A(2) / (den * den * (sg + eps));
      const bool ok = (!causal || sj <= i) && i < T_ && sj < T_ && key_ok(a, b, sj);
      sm.p[sr][c] = ok ? p : A(0);
      sm.s[sr][c] = ok ? p * g * (dp - sm.r1[c]) : A(0);
    }
    __syncthreads();
    for (int c = 0; c < TB; ++c) {
      const A p = sm.p[r][c], ds = sm.s[r][c];
#pragma unroll
      for (int m = 0; m < NO; ++m) {
        dv[m] = fma(p, sm.d[c][cl + TPR * m], dv[m]);   // backward.py:260
        dk[m] = fma(ds, sm.c[c][cl + TPR * m], dk[m]);  // backward.py:257
      }
    }
  }
  if (j < T_) {
    T* dkp = (T*)a.dk + b * a.sdk[0] + h * a.sdk[1] + (int64_t)j * a.sdk[2];
    T* dvp = (T*)a.dv + b * a.sdv[0] + h * a.sdv[1] + (int64_t)j * a.sdv[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + TPR * m;
      if (d < D) {
        dkp[d] = (T)(dk[m] * scale);
        dvp[d] = (T)dv[m];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

#define KAT_DMAX_SWITCH(D, ...)                                     \
  if ((D) <= 64) { constexpr int DM = 64; __VA_ARGS__; }            \
  else if ((D) <= 128) { constexpr int DM = 128; __VA_ARGS__; }     \
  else if ((D) <= 256) { constexpr int DM = 256; __VA_ARGS__; }     \
  else if ((D) <= 512) { constexpr int DM = 512; __VA_ARGS__; }     \
  else { constexpr int DM = 1024; __VA_ARGS__; }

template <typename T> static int tile_edge(int D) {
  constexpr int B = sizeof(typename AccT<T>::type);
  int tb = 0;
  KAT_DMAX_SWITCH(D, tb = gen_tb<B, DM>());
  return tb;
}

template <typename T> int attn_fwd_generic(const AttnArgs& a, hipStream_t st) {
  const int tb = tile_edge<T>(a.D);
  dim3 grid((a.T + tb - 1) / tb, a.B * a.H);
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_fwd_generic_k<T, DM>), grid, dim3(256), 0, st, a));
  return check_launch("kat_attn_fwd (tiled)");
}

template <typename T>
int attn_delta(const AttnArgs& a, typename AccT<T>::type* delta, typename AccT<T>::type* cinv, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  const bool vec = a.D % (16 / (int)sizeof(T)) == 0 && aligned16(a.o) && aligned16(a.dout) &&
                   (a.so[0] * (int64_t)sizeof(T)) % 16 == 0 && (a.so[1] * (int64_t)sizeof(T)) % 16 == 0 &&
                   (a.so[2] * (int64_t)sizeof(T)) % 16 == 0 && (a.sdo[0] * (int64_t)sizeof(T)) % 16 == 0 &&
                   (a.sdo[1] * (int64_t)sizeof(T)) % 16 == 0 && (a.sdo[2] * (int64_t)sizeof(T)) % 16 == 0;
  if (vec)
    hipLaunchKernelGGL((attn_delta_k<T, true>), dim3((unsigned)((rows * 16 + 255) / 256)), dim3(256),
                       0, st, a, delta, cinv);
  else
    hipLaunchKernelGGL((attn_delta_k<T, false>), dim3((unsigned)((rows * 64 + 255) / 256)),
                       dim3(256), 0, st, a, delta, cinv);
  return check_launch("kat_attn_bwd (delta)");
}

template <typename T> int attn_bwd_generic(const AttnArgs& a, const typename AccT<T>::type* delta, hipStream_t st) {
  const int tb = tile_edge<T>(a.D);
  dim3 grid((a.T + tb - 1) / tb, a.B * a.H);
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_bwd_dq_generic_k<T, DM>), grid, dim3(256), 0, st,
                                          a, delta));
  if (int rc = check_launch("kat_attn_bwd (dq, tiled)")) return rc;
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_bwd_dkv_generic_k<T, DM>), grid, dim3(256), 0, st,
                                          a, delta));
  return check_launch("kat_attn_bwd (dkv, tiled)");
}

#define KAT_GENERIC_INST(T)                                                                      \
  template int attn_fwd_generic<T>(const AttnArgs&, hipStream_t);                                \
  template int attn_delta<T>(const AttnArgs&, AccT<T>::type*, AccT<T>::type*, hipStream_t);      \
  template int attn_bwd_generic<T>(const AttnArgs&, const AccT<T>::type*, hipStream_t);
KAT_GENERIC_INST(float)
KAT_GENERIC_INST(bf16)
KAT_GENERIC_INST(f16)
KAT_GENERIC_INST(double)

}  // namespace kat
