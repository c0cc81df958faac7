// Rational attention on gfx950 -- fp32-exact tiled kernels.
//
// These kernels compute in fp32 FMA on the vector ALUs, with 32x32 query/key
// tiles staged through LDS. They serve fp32 (and fp64-free) inputs, head
// dims the MFMA kernels do not cover (any D <= 256), and are the
// independent on-GPU cross-check of the bf16 MFMA kernels.
//
// Math (reference forward.py:110-159, backward.py:116-154, 222-260):
//   s_ij = (q_i . k_j) * scale - slope_h * |i - j|,  j <= i (causal), every j
//   (causal == 0); keys the padding mask drops are skipped
//   f_ij = sigma(s_ij)^4, L_i = sum_j f_ij (stored without eps)
//   o_i  = sum_j f_ij v_j / (L_i + eps)
//   p = f / (L + eps), g = 2 / ((|s|+1)^2 (sigma + eps)), dS = p g (dO_i.v_j - Delta_i)
//   dq = scale * sum_j dS k_j,  dk = scale * sum_i dS q_i,  dv = sum_i p dO_i
// In causal mode keys j > i are never visited, exactly as the reference
// kernels' loops.

#include <algorithm>

#include "kat_common.h"
#include "kat_internal.h"
#include "attn_common.h"

namespace kat {

constexpr int GB = 32;  // tile edge (queries per block, keys per tile)

template <int DMAX> struct GenericTiles {
  float a[GB][DMAX + 1];  // Q (fwd, dq) or K (dkv)
  float b[GB][DMAX + 1];  // K (fwd, dq) or V (dkv)
  float c[GB][DMAX + 1];  // V (fwd), dO (dq), Q (dkv)
  float d[GB][DMAX + 1];  // unused (fwd), V (dq), dO (dkv)
  float p[GB][GB + 1];    // f / p tile
  float s[GB][GB + 1];    // dS tile
  float r0[GB], r1[GB];   // per-row L / Delta
};

template <typename T, int DMAX>
__device__ __forceinline__ void load_tile(float (*dst)[DMAX + 1], const T* __restrict__ src,
                                          int64_t st, int row0, int n_rows, int D) {
  for (int idx = threadIdx.x; idx < GB * DMAX; idx += blockDim.x) {
    const int r = idx / DMAX, d = idx - r * DMAX;
    float val = 0.f;
    if (d < D && row0 + r < n_rows) val = (float)src[(int64_t)(row0 + r) * st + d];
    dst[r][d] = val;
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_fwd_generic_k(AttnArgs a) {
  __shared__ GenericTiles<DMAX> sm;
  constexpr int NO = DMAX / 8;  // output columns per thread
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int q0 = blockIdx.x * GB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const float slope = a.slopes[h];
  const int tid = threadIdx.x, r = tid >> 3, cl = tid & 7;
  const int i = q0 + r;

  load_tile<T, DMAX>(sm.a, q, a.sq[2], q0, T_, D);
  float acc[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) acc[m] = 0.f;
  float l = 0.f;
  const bool causal = a.causal != 0;
  const int kend = causal ? std::min(q0 + GB, T_) : T_;  // causal: keys < q0 + GB
  for (int k0 = 0; k0 < kend; k0 += GB) {
    __syncthreads();
    load_tile<T, DMAX>(sm.b, k, a.sk[2], k0, T_, D);
    load_tile<T, DMAX>(sm.c, v, a.sv[2], k0, T_, D);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = cl + 8 * m, j = k0 + c;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(sm.a[r][d], sm.b[c][d], dot);
      const float s = dot * a.scale - slope * fabsf((float)(i - j));  // forward.py:129-133
      const float sg = rsig(s);                                       // forward.py:137-140
      const float s2 = sg * sg;
      const bool vis = (causal ? j <= i : j < T_) && i < T_ && key_ok(a, b, j);
      sm.p[r][c] = vis ? s2 * s2 : 0.f;
    }
    __syncthreads();
    for (int c = 0; c < GB; ++c) {
      const float f = sm.p[r][c];
      l += f;  // forward.py:142
#pragma unroll
      for (int m = 0; m < NO; ++m) acc[m] = fmaf(f, sm.c[c][cl + 8 * m], acc[m]);  // :147
    }
  }
  if (i < T_) {
    const float inv = 1.f / (l + a.eps);  // forward.py:150
    T* o = (T*)a.o + b * a.so[0] + h * a.so[1] + (int64_t)i * a.so[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + 8 * m;
      if (d < D) o[d] = (T)(acc[m] * inv);
    }
    if (cl == 0) a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)i * a.sl[2]] = l;  // :159
  }
}

// Delta_i = <dO_i, O_i> (backward.py:117) and cinv_i = 1 / (16 (L_i + eps)).
// 16 lanes per row, 16-byte loads (VEC16) or one wave per row, scalar loads.
template <typename T, bool VEC16>
__global__ __launch_bounds__(256) void attn_delta_k(AttnArgs a, float* __restrict__ delta,
                                                    float* __restrict__ cinv) {
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
  float s = 0.f;
  if (live) {
    for (int d = sub * V; d < a.D; d += LPR * V) {
      float ov[V], gv[V];
      load_acc<T, V>(o + d, ov);
      load_acc<T, V>(dO + d, gv);
#pragma unroll
      for (int e = 0; e < V; ++e) s = fmaf(gv[e], ov[e], s);
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (live && sub == 0) {
    delta[row] = s;
    const float l = a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)i * a.sl[2]];
    cinv[row] = 1.f / (16.f * (l + a.eps));
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_bwd_dq_generic_k(AttnArgs a,
                                                             const float* __restrict__ delta) {
  __shared__ GenericTiles<DMAX> sm;
  constexpr int NO = DMAX / 8;
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int q0 = blockIdx.x * GB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* dO = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float slope = a.slopes[h];
  const int tid = threadIdx.x, r = tid >> 3, cl = tid & 7;
  const int i = q0 + r;

  load_tile<T, DMAX>(sm.a, q, a.sq[2], q0, T_, D);
  load_tile<T, DMAX>(sm.c, dO, a.sdo[2], q0, T_, D);
  if (tid < GB) {
    const int ii = q0 + tid;
    sm.r0[tid] = ii < T_ ? a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)ii * a.sl[2]] : 0.f;
    sm.r1[tid] = ii < T_ ? delta[((int64_t)bh) * T_ + ii] : 0.f;
  }
  float acc[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) acc[m] = 0.f;
  const bool causal = a.causal != 0;
  const int kend = causal ? std::min(q0 + GB, T_) : T_;
  for (int k0 = 0; k0 < kend; k0 += GB) {
    __syncthreads();
    load_tile<T, DMAX>(sm.b, k, a.sk[2], k0, T_, D);
    load_tile<T, DMAX>(sm.d, v, a.sv[2], k0, T_, D);
    __syncthreads();
    const float Li = sm.r0[r], Di = sm.r1[r];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = cl + 8 * m, j = k0 + c;
      float dot = 0.f, dp = 0.f;
      for (int d = 0; d < D; ++d) {
        dot = fmaf(sm.a[r][d], sm.b[c][d], dot);
        dp = fmaf(sm.c[r][d], sm.d[c][d], dp);
      }
      // backward.py:133-151
      const float s = dot * a.scale - slope * fabsf((float)(i - j));
      const float den = fabsf(s) + 1.f;
      const float sg = 0.5f * (s / den + 1.f);
      const float s2 = sg * sg;
      const float p = s2 * s2 / (Li + a.eps);
      const float g = 2.f / (den * den * (sg + a.eps));
      const bool vis = (causal ? j <= i : j < T_) && i < T_ && key_ok(a, b, j);
      sm.s[r][c] = vis ? p * g * (dp - Di) : 0.f;
    }
    __syncthreads();
    for (int c = 0; c < GB; ++c) {
      const float ds = sm.s[r][c];
#pragma unroll
      for (int m = 0; m < NO; ++m) acc[m] = fmaf(ds, sm.b[c][cl + 8 * m], acc[m]);  // :154
    }
  }
  if (i < T_) {
    T* dq = (T*)a.dq + b * a.sdq[0] + h * a.sdq[1] + (int64_t)i * a.sdq[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + 8 * m;
      if (d < D) dq[d] = (T)(acc[m] * a.scale);
    }
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void attn_bwd_dkv_generic_k(AttnArgs a,
                                                              const float* __restrict__ delta) {
  __shared__ GenericTiles<DMAX> sm;
  constexpr int NO = DMAX / 8;
  const int H = a.H, T_ = a.T, D = a.D;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int k0 = blockIdx.x * GB;
  const T* q = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* k = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* v = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* dO = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float slope = a.slopes[h];
  const int tid = threadIdx.x, r = tid >> 3, cl = tid & 7;
  const int j = k0 + r;  // this thread's key row

  load_tile<T, DMAX>(sm.a, k, a.sk[2], k0, T_, D);
  load_tile<T, DMAX>(sm.b, v, a.sv[2], k0, T_, D);
  float dk[NO], dv[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) dk[m] = dv[m] = 0.f;
  const bool causal = a.causal != 0;
  const bool jok = j < T_ && key_ok(a, b, j);
  for (int q0 = causal ? (k0 / GB) * GB : 0; q0 < T_; q0 += GB) {  // causal: queries >= k0
    __syncthreads();
    load_tile<T, DMAX>(sm.c, q, a.sq[2], q0, T_, D);
    load_tile<T, DMAX>(sm.d, dO, a.sdo[2], q0, T_, D);
    if (tid < GB) {
      const int ii = q0 + tid;
      sm.r0[tid] = ii < T_ ? a.L[b * a.sl[0] + h * a.sl[1] + (int64_t)ii * a.sl[2]] : 0.f;
      sm.r1[tid] = ii < T_ ? delta[((int64_t)bh) * T_ + ii] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = cl + 8 * m, i = q0 + c;
      float dot = 0.f, dp = 0.f;
      for (int d = 0; d < D; ++d) {
        dot = fmaf(sm.c[c][d], sm.a[r][d], dot);
        dp = fmaf(sm.d[c][d], sm.b[r][d], dp);
      }
      // backward.py:233-254
      const float s = dot * a.scale - slope * fabsf((float)(i - j));
      const float den = fabsf(s) + 1.f;
      const float sg = 0.5f * (s / den + 1.f);
      const float s2 = sg * sg;
      const float p = s2 * s2 / (sm.r0[c] + a.eps);
      const float g = 2.f / (den * den * (sg + a.eps));
      const bool ok = (!causal || j <= i) && i < T_ && jok;
      sm.p[r][c] = ok ? p : 0.f;
      sm.s[r][c] = ok ? p * g * (dp - sm.r1[c]) : 0.f;
    }
    __syncthreads();
    for (int c = 0; c < GB; ++c) {
      const float p = sm.p[r][c], ds = sm.s[r][c];
#pragma unroll
      for (int m = 0; m < NO; ++m) {
        dv[m] = fmaf(p, sm.d[c][cl + 8 * m], dv[m]);   // backward.py:260
        dk[m] = fmaf(ds, sm.c[c][cl + 8 * m], dk[m]);  // backward.py:257
      }
    }
  }
  if (j < T_) {
    T* dkp = (T*)a.dk + b * a.sdk[0] + h * a.sdk[1] + (int64_t)j * a.sdk[2];
    T* dvp = (T*)a.dv + b * a.sdv[0] + h * a.sdv[1] + (int64_t)j * a.sdv[2];
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const int d = cl + 8 * m;
      if (d < D) {
        dkp[d] = (T)(dk[m] * a.scale);
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
  else { constexpr int DM = 256; __VA_ARGS__; }

template <typename T> int attn_fwd_generic(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.T + GB - 1) / GB, a.B * a.H);
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_fwd_generic_k<T, DM>), grid, dim3(256), 0, st, a));
  return check_launch("kat_attn_fwd (fp32 tiled)");
}

template <typename T> int attn_delta(const AttnArgs& a, float* delta, float* cinv, hipStream_t st) {
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

template <typename T> int attn_bwd_generic(const AttnArgs& a, const float* delta, hipStream_t st) {
  dim3 grid((a.T + GB - 1) / GB, a.B * a.H);
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_bwd_dq_generic_k<T, DM>), grid, dim3(256), 0, st,
                                          a, delta));
  if (int rc = check_launch("kat_attn_bwd (dq, fp32 tiled)")) return rc;
  KAT_DMAX_SWITCH(a.D, hipLaunchKernelGGL((attn_bwd_dkv_generic_k<T, DM>), grid, dim3(256), 0, st,
                                          a, delta));
  return check_launch("kat_attn_bwd (dkv, fp32 tiled)");
}

template int attn_fwd_generic<float>(const AttnArgs&, hipStream_t);
template int attn_fwd_generic<bf16>(const AttnArgs&, hipStream_t);
template int attn_fwd_generic<f16>(const AttnArgs&, hipStream_t);
template int attn_delta<float>(const AttnArgs&, float*, float*, hipStream_t);
template int attn_delta<bf16>(const AttnArgs&, float*, float*, hipStream_t);
template int attn_delta<f16>(const AttnArgs&, float*, float*, hipStream_t);
template int attn_bwd_generic<float>(const AttnArgs&, const float*, hipStream_t);
template int attn_bwd_generic<bf16>(const AttnArgs&, const float*, hipStream_t);
template int attn_bwd_generic<f16>(const AttnArgs&, const float*, hipStream_t);

}  // namespace kat
