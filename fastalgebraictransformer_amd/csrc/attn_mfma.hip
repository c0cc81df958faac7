// bf16 / fp16 MFMA rational attention for gfx950 (CDNA4).
//
// Forward (one block = 128 queries of one (b, h); 4 waves x 32 queries):
//   for each 64-key tile (K, V row-major in LDS, double-buffered, padded rows):
//     S^T[key][q] = K . Q^T             v_mfma_f32_16x16x32_{bf16,f16}
//       A = K rows from LDS (ds_read_b128), B = Q^T fragments kept in VGPRs,
//       C initialised with the ALiBi bias / scale, so one FMA gives
//       s = scale * q.k - slope * (q - key)
//     f' = (1 + s / (|s| + 1))^4 = 16 sigma(s)^4     (one v_rcp_f32 per score)
//     O^T[d][q] += V^T . P^T            A = V^T via ds_read_tr16_b64 from the
//                                       row-major V tile, B = P^T straight from
//                                       the S^T accumulator registers
//   L' = sum f' (per lane, then across the 4 lane groups),
//   o = O / (L' + 16 eps), L = L' / 16.
// The factor 16 is exact in binary floating point, so o and L equal the
// reference's f = sigma^4 formulation (forward.py:137-159) up to rounding.
// There is no running-max rescale: sigma^4 lies in (0, 1).
//
// MFMA 16x16x32 operand layout (lane l, g = l / 16): A[m = l % 16][k-set of g],
// B[k-set of g][n = l % 16], C[4g + j][l % 16]. A and B use the same k-set per
// lane group, so any consistent assignment of keys to (g, element) is valid;
// here lane group g, element i < 4 holds key 4g + i of the first 16-key
// subtile and element 4 + i key 4g + i of the second.

#include <algorithm>
#include <type_traits>

#include "attn_common.h"
#include "kat_common.h"
#include "kat_internal.h"

namespace kat {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 mma(const i16x8& a, const i16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8)a, (bf16x8)b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 f = {x, y};
    bf16x2 b = __builtin_convertvector(f, bf16x2);
    return __builtin_bit_cast(uint32_t, b);
  }
};
template <> struct Mfma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x4 mma(const i16x8& a, const i16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16((f16x8)a, (f16x8)b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 f = {x, y};
    f16x2 b = __builtin_convertvector(f, f16x2);
    return __builtin_bit_cast(uint32_t, b);
  }
};

// Block order. Workgroups are dispatched round-robin over the 8 XCDs (block
// id i runs on XCD i % 8), and each XCD has its own L2. Heads are assigned to
// XCDs (head h on XCD h % 8, when B*H is a multiple of 8) and each XCD walks
// its heads one after another, longest (causal) tiles first, so the K/V (or
// Q/dO) of the one or two heads in flight per XCD stay L2-resident.
// Returns the (b*H + h) index and the tile rank (0 = most work).
__device__ __forceinline__ void block_order(int id, int n_tiles, int BH, int& bh, int& rank) {
  if ((BH & 7) == 0) {
    const int xcd = id & 7, slot = id >> 3;
    const int hl = slot / n_tiles;
    rank = slot - hl * n_tiles;
    bh = xcd + 8 * hl;
  } else {
    bh = id / n_tiles;
    rank = id - bh * n_tiles;
  }
}

constexpr int FBM = 128;  // queries per block
constexpr int FBN = 64;   // keys per tile
constexpr int FWAVES = 4;

template <int D> struct FwdSmem {
  static constexpr int LD = D + 16;  // padded row (elements): spreads rows over banks
  short k[2][FBN * LD];
  short v[2][FBN * LD];
};

__device__ __forceinline__ i16x8 lds_read16(const short* p) {
  return *reinterpret_cast<const i16x8*>(p);
}

// Transposing LDS read (gfx950): within each 16-lane group, result lane i,
// element j = the 16-bit element (i % 4) of the 8 bytes addressed by source
// lane i / 4 + 4 j. With source lane s addressing row (r0 + s / 4), column
// (c0 + 4 (s % 4)) of a row-major tile, lane i receives rows r0..r0+3 at
// column c0 + i.
__device__ __forceinline__ i16x4 lds_read_tr(const short* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// fp16 products for dS: dS = p g (dP - Delta) is rounded to fp16 (11-bit
// significand) rather than bf16 before the dQ = dS K and dK = dS^T Q
// products, so its rounding error is 4x smaller; the K / Q operands of those
// products are converted bf16 -> fp16, which is exact for |x| in
// [2^-14, 65504]. Larger magnitudes are clamped to +-65504, and smaller ones
// keep fp16's subnormal spacing 2^-24.
__device__ __forceinline__ f32x4 mma_f16(const i16x8& a, const i16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16((f16x8)a, (f16x8)b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack2_f16(float x, float y) { return Mfma<f16>::pack2(x, y); }

template <typename T> __device__ __forceinline__ i16x8 frag_to_f16(const i16x8& v);
template <> __device__ __forceinline__ i16x8 frag_to_f16<f16>(const i16x8& v) { return v; }
template <> __device__ __forceinline__ i16x8 frag_to_f16<bf16>(const i16x8& v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = __builtin_bit_cast(u32x4, v);
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __builtin_bit_cast(float, w[e] << 16);
    const float hi = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    o[e] = pack2_f16(fminf(fmaxf(lo, -65504.f), 65504.f), fminf(fmaxf(hi, -65504.f), 65504.f));
  }
  return __builtin_bit_cast(i16x8, o);
}

// Shared pieces of the forward and dQ kernels: 64-key K/V tiles staged
// global -> VGPRs -> LDS (double-buffered), rows zero-filled past T.
template <typename T, int D> struct KvStager {
  static constexpr int LD = FwdSmem<D>::LD;
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int LOADS = FBN * CPR / 256;     // chunks per thread per tile
  i16x8 kst[LOADS], vst[LOADS];
  __device__ __forceinline__ void load(const T* __restrict__ kp, int64_t skt,
                                       const T* __restrict__ vp, int64_t svt, int k0, int T_,
                                       int tid) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      const int row = c / CPR, col = (c % CPR) * 8;
      const int key = k0 + row;
      if (key < T_) {
        kst[u] = *reinterpret_cast<const i16x8*>(kp + (int64_t)key * skt + col);
        vst[u] = *reinterpret_cast<const i16x8*>(vp + (int64_t)key * svt + col);
      } else {
        kst[u] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
        vst[u] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  }
  __device__ __forceinline__ void store(FwdSmem<D>& sm, int buf, int tid) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      const int row = c / CPR, col = (c % CPR) * 8;
      *reinterpret_cast<i16x8*>(&sm.k[buf][row * LD + col]) = kst[u];
      *reinterpret_cast<i16x8*>(&sm.v[buf][row * LD + col]) = vst[u];
    }
  }
};

// A-operand fragment of a 16x16x32 MFMA taken transposed from a row-major
// [row][col] LDS tile: lane (g, li) receives column c0 + li of rows
// r0 + 4 g + {0..3} (elements 0-3) and r0 + 16 + 4 g + {0..3} (elements 4-7).
__device__ __forceinline__ i16x8 lds_frag_tr(const short* tile, int ld, int r0, int c0, int g,
                                             int li) {
  const short* p0 = tile + (r0 + 4 * g + (li >> 2)) * ld + c0 + 4 * (li & 3);
  const i16x4 lo = lds_read_tr(p0);
  const i16x4 hi = lds_read_tr(p0 + 16 * ld);
  return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_mfma_k(AttnArgs a) {
  typedef Mfma<T> M;
  constexpr int LD = FwdSmem<D>::LD;
  constexpr int KK = D / 32;   // k-steps of QK^T
  constexpr int DS = D / 16;   // 16-wide d subtiles of O^T
  __shared__ FwdSmem<D> sm;

  const int T_ = a.T, H = a.H;
  const int n_qt = (T_ + FBM - 1) / FBM;
  int bh, rank;
  block_order((int)blockIdx.x, n_qt, a.B * H, bh, rank);
  const int qt = n_qt - 1 - rank;  // longest (causal) tiles first
  const int b = bh / H, h = bh - b * H;
  const int q0 = qt * FBM;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qw = q0 + 32 * w;  // first query of this wave

  const T* __restrict__ qp = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* __restrict__ kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* __restrict__ vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const float slope = a.slopes[h];
  const float scale = a.scale;

  // Q^T fragments (B operand): lane (g, li) holds Q[qw + 16 qs + li][32 kk + 8 g .. +7]
  i16x8 qf[2][KK];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int qrow = qw + 16 * qs + li;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      qf[qs][kk] = qrow < T_
                       ? *reinterpret_cast<const i16x8*>(qp + (int64_t)qrow * a.sq[2] + 32 * kk + 8 * g)
                       : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  // ALiBi bias slope * (key - q) split into a per-lane part, fed to QK^T as its
  // C input (divided by scale), and a wave-uniform part added by the FMA that
  // applies the scale: element (qs, ks, j) has key = k0 + 16 ks + 4 g + j and
  // q = qw + 16 qs + li.
  f32x4 cb;
#pragma unroll
  for (int j = 0; j < 4; ++j) cb[j] = (slope / scale) * (float)(4 * g + j - li);

  f32x4 oacc[DS][2];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) oacc[ds][qs] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lsum[2] = {0.f, 0.f};

  // one 64-key tile; MASK: the tile crosses this wave's diagonal
  auto tile = [&](auto mask_tag, int k0, const short* ks_, const short* vs_) {
    constexpr bool MASK = decltype(mask_tag)::value;
    // S^T = K Q^T (+ bias / scale): k-step outer, 8 independent accumulators
    f32x4 sacc[2][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) sacc[qs][ks] = cb;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      i16x8 kf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[ks] = lds_read16(ks_ + (16 * ks + li) * LD + 32 * kk + 8 * g);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) sacc[qs][ks] = M::mma(kf[ks], qf[qs][kk], sacc[qs][ks]);
    }
    // f' = (1 + s r)^4, r = 1 / (|s| + 1); P^T packed straight from the
    // accumulator layout into the B operand of O^T += V^T P^T
    i16x8 pf[2][2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      float ls = 0.f;
      uint32_t pk[4][2];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float tterm = slope * (float)(k0 - qw + 16 * ks - 16 * qs);
        float f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = fmaf(sacc[qs][ks][j], scale, tterm);
          const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
          const float t = fmaf(s, r, 1.f);
          const float t2 = t * t;
          f[j] = t2 * t2;
          if (MASK && k0 + 16 * ks + 4 * g + j > qw + 16 * qs + li) f[j] = 0.f;
        }
        ls += (f[0] + f[1]) + (f[2] + f[3]);
        pk[ks][0] = M::pack2(f[0], f[1]);
        pk[ks][1] = M::pack2(f[2], f[3]);
      }
      lsum[qs] += ls;
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 u = {pk[2 * kk2][0], pk[2 * kk2][1], pk[2 * kk2 + 1][0], pk[2 * kk2 + 1][1]};
        pf[qs][kk2] = __builtin_bit_cast(i16x8, u);
      }
    }
    // O^T += V^T P^T, two d-subtiles at a time (4 independent chains)
#pragma unroll
    for (int ds = 0; ds < DS; ds += 2) {
      i16x8 vf[2][2];
#pragma unroll
      for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int kk2 = 0; kk2 < 2; ++kk2) vf[dd][kk2] = lds_frag_tr(vs_, LD, 32 * kk2, 16 * (ds + dd), g, li);
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2)
#pragma unroll
        for (int dd = 0; dd < 2; ++dd)
#pragma unroll
          for (int qs = 0; qs < 2; ++qs)
            oacc[ds + dd][qs] = M::mma(vf[dd][kk2], pf[qs][kk2], oacc[ds + dd][qs]);
    }
  };

  const int kend = std::min(q0 + FBM, T_);
  const int n_kt = (kend + FBN - 1) / FBN;
  KvStager<T, D> stg;
  stg.load(kp, a.sk[2], vp, a.sv[2], 0, T_, tid);
  stg.store(sm, 0, tid);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < n_kt;
    if (more) stg.load(kp, a.sk[2], vp, a.sv[2], (kt + 1) * FBN, T_, tid);
    const int k0 = kt * FBN;
    if (k0 + FBN - 1 <= qw)
      tile(std::false_type{}, k0, sm.k[buf], sm.v[buf]);
    else if (k0 <= qw + 31)
      tile(std::true_type{}, k0, sm.k[buf], sm.v[buf]);
    if (more) stg.store(sm, buf ^ 1, tid);
    __syncthreads();
  }

  // epilogue: L' across the 4 lane groups, normalise, store
  T* __restrict__ op = (T*)a.o + b * a.so[0] + h * a.so[1];
  float* __restrict__ Lp = a.L + b * a.sl[0] + h * a.sl[1];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    float l = lsum[qs];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qrow = qw + 16 * qs + li;
    const float inv = 1.f / (l + 16.f * a.eps);
    if (qrow < T_) {
      if (g == 0) Lp[(int64_t)qrow * a.sl[2]] = l * 0.0625f;
      T* orow = op + (int64_t)qrow * a.so[2];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const f32x4 o = oacc[ds][qs];
        u32x2 u = {M::pack2(o[0] * inv, o[1] * inv), M::pack2(o[2] * inv, o[3] * inv)};
        *reinterpret_cast<u32x2*>(orow + 16 * ds + 4 * g) = u;
      }
    }
  }
}

// ============================================================================
// Backward.  Per score (j <= i), with t = 1 + s r, r = 1 / (|s| + 1)
// (so sigma = t / 2) and cinv_i = 1 / (16 (L_i + eps)):
//   p  = sigma^4 / (L_i + eps)                 = t^4 cinv_i
//   dS = p g (dP - Delta_i), g = 2 r^2 / sigma = 4 cinv_i t^3 r^2 (dP - Delta_i)
// The reference writes g = 2 / ((|s|+1)^2 (sigma + eps)) (backward.py:145);
// these kernels use sigma in place of sigma + eps, a relative change of
// eps / (sigma + eps) in dS: <= 2e-6 wherever s >= 0, and otherwise on scores
// whose p <= (r / 2)^4 / L is itself negligible.
//   dQ  = scale dS K      -- attn_bwd_dq_mfma_k   (query-tile blocks)
//   dK  = scale dS^T Q    -- attn_bwd_dkv_mfma_k  (key-tile blocks)
//   dV  = P^T dO
// Both kernels recompute S (and dP); no atomics, so results are deterministic.
// dS enters the dQ and dK products in fp16 (see frag_to_f16).
// ============================================================================

// dQ: mirrors the forward (128 queries per block, 64-key K/V tiles in LDS).
//   S^T  = K Q^T (+bias)   A = K  (LDS, b128)      B = Q^T  (VGPRs)
//   dP^T = V dO^T          A = V  (LDS, b128)      B = dO^T (VGPRs)
//   dQ^T += K^T dS^T       A = K^T (LDS, transposing read)  B = dS^T (registers)
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_mfma_k(AttnArgs a,
                                                         const float* __restrict__ delta,
                                                         const float* __restrict__ cinv) {
  typedef Mfma<T> M;
  constexpr int LD = FwdSmem<D>::LD;
  constexpr int KK = D / 32;
  constexpr int DS = D / 16;
  __shared__ FwdSmem<D> sm;

  const int T_ = a.T, H = a.H;
  const int n_qt = (T_ + FBM - 1) / FBM;
  int bh, rank;
  block_order((int)blockIdx.x, n_qt, a.B * H, bh, rank);
  const int qt = n_qt - 1 - rank;
  const int b = bh / H, h = bh - b * H;
  const int q0 = qt * FBM;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qw = q0 + 32 * w;

  const T* __restrict__ qp = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* __restrict__ kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* __restrict__ vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* __restrict__ dop = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float slope = a.slopes[h];
  const float scale = a.scale;

  i16x8 qf[2][KK], dof[2][KK];
  float c4[2], nc4d[2];  // 4 cinv_q and -4 cinv_q Delta_q for q = qw + 16 qs + li
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int qrow = qw + 16 * qs + li;
    const bool ok = qrow < T_;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qf[qs][kk] = ok ? *reinterpret_cast<const i16x8*>(qp + (int64_t)qrow * a.sq[2] + 32 * kk + 8 * g)
                      : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
      dof[qs][kk] = ok ? *reinterpret_cast<const i16x8*>(dop + (int64_t)qrow * a.sdo[2] + 32 * kk + 8 * g)
                       : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    const int64_t ri = (int64_t)bh * T_ + qrow;
    c4[qs] = ok ? 4.f * cinv[ri] : 0.f;
    nc4d[qs] = ok ? -c4[qs] * delta[ri] : 0.f;
  }
  f32x4 cb;
#pragma unroll
  for (int j = 0; j < 4; ++j) cb[j] = (slope / scale) * (float)(4 * g + j - li);

  f32x4 dqacc[DS][2];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) dqacc[ds][qs] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto tile = [&](auto mask_tag, int k0, const short* ks_, const short* vs_) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x4 sacc[2][4], pacc[2][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        sacc[qs][ks] = cb;
        pacc[qs][ks] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      i16x8 kf[4], vf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        kf[ks] = lds_read16(ks_ + (16 * ks + li) * LD + 32 * kk + 8 * g);
        vf[ks] = lds_read16(vs_ + (16 * ks + li) * LD + 32 * kk + 8 * g);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
          sacc[qs][ks] = M::mma(kf[ks], qf[qs][kk], sacc[qs][ks]);
          pacc[qs][ks] = M::mma(vf[ks], dof[qs][kk], pacc[qs][ks]);
        }
    }
    i16x8 dsf[2][2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      uint32_t pk[4][2];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float tterm = slope * (float)(k0 - qw + 16 * ks - 16 * qs);
        float d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = fmaf(sacc[qs][ks][j], scale, tterm);
          const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
          const float t = fmaf(s, r, 1.f);
          const float u = t * r;
          d[j] = (u * u * t) * fmaf(pacc[qs][ks][j], c4[qs], nc4d[qs]);
          if (MASK && k0 + 16 * ks + 4 * g + j > qw + 16 * qs + li) d[j] = 0.f;
        }
        pk[ks][0] = pack2_f16(d[0], d[1]);
        pk[ks][1] = pack2_f16(d[2], d[3]);
      }
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 uu = {pk[2 * kk2][0], pk[2 * kk2][1], pk[2 * kk2 + 1][0], pk[2 * kk2 + 1][1]};
        dsf[qs][kk2] = __builtin_bit_cast(i16x8, uu);
      }
    }
#pragma unroll
    for (int ds = 0; ds < DS; ds += 2) {
      i16x8 kt[2][2];
#pragma unroll
      for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int kk2 = 0; kk2 < 2; ++kk2)
          kt[dd][kk2] = frag_to_f16<T>(lds_frag_tr(ks_, LD, 32 * kk2, 16 * (ds + dd), g, li));
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2)
#pragma unroll
        for (int dd = 0; dd < 2; ++dd)
#pragma unroll
          for (int qs = 0; qs < 2; ++qs)
            dqacc[ds + dd][qs] = mma_f16(kt[dd][kk2], dsf[qs][kk2], dqacc[ds + dd][qs]);
    }
  };

  const int kend = std::min(q0 + FBM, T_);
  const int n_kt = (kend + FBN - 1) / FBN;
  KvStager<T, D> stg;
  stg.load(kp, a.sk[2], vp, a.sv[2], 0, T_, tid);
  stg.store(sm, 0, tid);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < n_kt;
    if (more) stg.load(kp, a.sk[2], vp, a.sv[2], (kt + 1) * FBN, T_, tid);
    const int k0 = kt * FBN;
    if (k0 + FBN - 1 <= qw)
      tile(std::false_type{}, k0, sm.k[buf], sm.v[buf]);
    else if (k0 <= qw + 31)
      tile(std::true_type{}, k0, sm.k[buf], sm.v[buf]);
    if (more) stg.store(sm, buf ^ 1, tid);
    __syncthreads();
  }

  T* __restrict__ dqp = (T*)a.dq + b * a.sdq[0] + h * a.sdq[1];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int qrow = qw + 16 * qs + li;
    if (qrow < T_) {
      T* row = dqp + (int64_t)qrow * a.sdq[2];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const f32x4 o = dqacc[ds][qs];
        u32x2 uu = {M::pack2(o[0] * scale, o[1] * scale), M::pack2(o[2] * scale, o[3] * scale)};
        *reinterpret_cast<u32x2*>(row + 16 * ds + 4 * g) = uu;
      }
    }
  }
}

// dK, dV: 128 keys per block (4 waves x 32 keys); 64-query Q / dO tiles in LDS,
// processed in two 32-query halves.
//   S  = Q K^T (+bias)    A = Q  (LDS, b128)               B = K^T (VGPRs)
//   dP = dO V^T           A = dO (LDS, b128)               B = V^T (VGPRs)
//   dV^T += dO^T P        A = dO^T (LDS, transposing read) B = P  (registers)
//   dK^T += Q^T dS        A = Q^T  (LDS, transposing read) B = dS (registers)
constexpr int KBN = 128;  // keys per block
constexpr int KBQ = 64;   // queries per LDS tile

template <int D> struct DkvSmem {
  static constexpr int LD = D + 16;
  short q[2][KBQ * LD];
  short o[2][KBQ * LD];  // dO
  float c4[2][KBQ];      // 4 cinv_q
  float nc4d[2][KBQ];    // -4 cinv_q Delta_q
};

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_dkv_mfma_k(AttnArgs a,
                                                          const float* __restrict__ delta,
                                                          const float* __restrict__ cinv) {
  typedef Mfma<T> M;
  constexpr int LD = DkvSmem<D>::LD;
  constexpr int KK = D / 32;
  constexpr int DS = D / 16;
  constexpr int CPR = D / 8;
  constexpr int LOADS = KBQ * CPR / 256;
  __shared__ DkvSmem<D> sm;

  const int T_ = a.T, H = a.H;
  const int n_kb = (T_ + KBN - 1) / KBN;
  int bh, kb;
  block_order((int)blockIdx.x, n_kb, a.B * H, bh, kb);  // kb 0 has the most query tiles
  const int b = bh / H, h = bh - b * H;
  const int k0 = kb * KBN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int kw = k0 + 32 * w;

  const T* __restrict__ qp = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* __restrict__ kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* __restrict__ vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* __restrict__ dop = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float* __restrict__ dl = delta + (int64_t)bh * T_;
  const float* __restrict__ ci = cinv + (int64_t)bh * T_;
  const float slope = a.slopes[h];
  const float scale = a.scale;

  // K^T / V^T fragments (B operands): lane (g, li) holds row kw + 16 ks + li,
  // columns 32 kk + 8 g .. +7
  i16x8 kf[2][KK], vf[2][KK];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int key = kw + 16 * ks + li;
    const bool ok = key < T_;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      kf[ks][kk] = ok ? *reinterpret_cast<const i16x8*>(kp + (int64_t)key * a.sk[2] + 32 * kk + 8 * g)
                      : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
      vf[ks][kk] = ok ? *reinterpret_cast<const i16x8*>(vp + (int64_t)key * a.sv[2] + 32 * kk + 8 * g)
                      : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  // S layout: lane (g, li) element j holds q = qh + 16 qs + 4 g + j,
  // key = kw + 16 ks + li; bias slope * (key - q) = per-lane part + uniform part
  f32x4 cb;
#pragma unroll
  for (int j = 0; j < 4; ++j) cb[j] = (slope / scale) * (float)(li - 4 * g - j);

  f32x4 dkacc[DS][2], dvacc[DS][2];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      dkacc[ds][ks] = f32x4{0.f, 0.f, 0.f, 0.f};
      dvacc[ds][ks] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  // one 32-query half (queries qh .. qh + 31) of the LDS tile; MASK: some
  // pair of the half has key > q
  auto half = [&](auto mask_tag, int qh, int r0, const short* qs_, const short* os_,
                  const float* c4s, const float* nds) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x4 sacc[2][2], pacc[2][2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        sacc[qs][ks] = cb;
        pacc[qs][ks] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      i16x8 qa[2], oa[2];
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        const int row = r0 + 16 * qs + li;
        qa[qs] = lds_read16(qs_ + row * LD + 32 * kk + 8 * g);
        oa[qs] = lds_read16(os_ + row * LD + 32 * kk + 8 * g);
      }
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          sacc[qs][ks] = M::mma(qa[qs], kf[ks][kk], sacc[qs][ks]);
          pacc[qs][ks] = M::mma(oa[qs], vf[ks][kk], pacc[qs][ks]);
        }
    }
    uint32_t ppk[2][2][2], dpk[2][2][2];  // [ks][qs][pair]
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const f32x4 c4v = *reinterpret_cast<const f32x4*>(c4s + r0 + 16 * qs + 4 * g);
      const f32x4 ndv = *reinterpret_cast<const f32x4*>(nds + r0 + 16 * qs + 4 * g);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float tterm = slope * (float)(kw + 16 * ks - qh - 16 * qs);
        float pv[4], dv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = fmaf(sacc[qs][ks][j], scale, tterm);
          const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
          const float t = fmaf(s, r, 1.f);
          const float t2 = t * t;
          const float u = t * r;
          pv[j] = (t2 * t2) * (0.25f * c4v[j]);
          dv[j] = (u * u * t) * fmaf(pacc[qs][ks][j], c4v[j], ndv[j]);
          if (MASK && kw + 16 * ks + li > qh + 16 * qs + 4 * g + j) {
            pv[j] = 0.f;
            dv[j] = 0.f;
          }
        }
        ppk[ks][qs][0] = M::pack2(pv[0], pv[1]);
        ppk[ks][qs][1] = M::pack2(pv[2], pv[3]);
        dpk[ks][qs][0] = pack2_f16(dv[0], dv[1]);
        dpk[ks][qs][1] = pack2_f16(dv[2], dv[3]);
      }
    }
    i16x8 pf[2], dsf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      u32x4 u1 = {ppk[ks][0][0], ppk[ks][0][1], ppk[ks][1][0], ppk[ks][1][1]};
      u32x4 u2 = {dpk[ks][0][0], dpk[ks][0][1], dpk[ks][1][0], dpk[ks][1][1]};
      pf[ks] = __builtin_bit_cast(i16x8, u1);
      dsf[ks] = __builtin_bit_cast(i16x8, u2);
    }
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const i16x8 ot = lds_frag_tr(os_, LD, r0, 16 * ds, g, li);
      const i16x8 qtr = frag_to_f16<T>(lds_frag_tr(qs_, LD, r0, 16 * ds, g, li));
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        dvacc[ds][ks] = M::mma(ot, pf[ks], dvacc[ds][ks]);
        dkacc[ds][ks] = mma_f16(qtr, dsf[ks], dkacc[ds][ks]);
      }
    }
  };

  const int qstart = k0;  // causal: queries >= first key of the block
  const int n_qt = qstart < T_ ? (T_ - qstart + KBQ - 1) / KBQ : 0;
  i16x8 qst[LOADS], ost[LOADS];
  float cst = 0.f, dst = 0.f;
  auto load_tile = [&](int it) {
    const int q0 = qstart + it * KBQ;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      const int row = c / CPR, col = (c % CPR) * 8;
      const int qr = q0 + row;
      if (qr < T_) {
        qst[u] = *reinterpret_cast<const i16x8*>(qp + (int64_t)qr * a.sq[2] + col);
        ost[u] = *reinterpret_cast<const i16x8*>(dop + (int64_t)qr * a.sdo[2] + col);
      } else {
        qst[u] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
        ost[u] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    if (tid < KBQ) {
      const int qr = q0 + tid;
      const float c = qr < T_ ? 4.f * ci[qr] : 0.f;
      cst = c;
      dst = qr < T_ ? -c * dl[qr] : 0.f;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      const int row = c / CPR, col = (c % CPR) * 8;
      *reinterpret_cast<i16x8*>(&sm.q[buf][row * LD + col]) = qst[u];
      *reinterpret_cast<i16x8*>(&sm.o[buf][row * LD + col]) = ost[u];
    }
    if (tid < KBQ) {
      sm.c4[buf][tid] = cst;
      sm.nc4d[buf][tid] = dst;
    }
  };

  if (n_qt > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int it = 0; it < n_qt; ++it) {
    const int buf = it & 1;
    const bool more = it + 1 < n_qt;
    if (more) load_tile(it + 1);
    const int q0 = qstart + it * KBQ;
    const short* qs_ = sm.q[buf];
    const short* os_ = sm.o[buf];
    const float* c4s = sm.c4[buf];
    const float* nds = sm.nc4d[buf];
    if (q0 >= kw + 31) {  // every pair of the tile has key <= q
      half(std::false_type{}, q0, 0, qs_, os_, c4s, nds);
      half(std::false_type{}, q0 + 32, 32, qs_, os_, c4s, nds);
    } else {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int qh = q0 + 32 * h2;
        if (qh + 31 < kw) continue;  // every pair of the half has key > q
        if (qh >= kw + 31)
          half(std::false_type{}, qh, 32 * h2, qs_, os_, c4s, nds);
        else
          half(std::true_type{}, qh, 32 * h2, qs_, os_, c4s, nds);
      }
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  T* __restrict__ dkp = (T*)a.dk + b * a.sdk[0] + h * a.sdk[1];
  T* __restrict__ dvp = (T*)a.dv + b * a.sdv[0] + h * a.sdv[1];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int key = kw + 16 * ks + li;
    if (key < T_) {
      T* rk = dkp + (int64_t)key * a.sdk[2];
      T* rv = dvp + (int64_t)key * a.sdv[2];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const f32x4 kq = dkacc[ds][ks];
        const f32x4 vq = dvacc[ds][ks];
        u32x2 uk = {M::pack2(kq[0] * scale, kq[1] * scale), M::pack2(kq[2] * scale, kq[3] * scale)};
        u32x2 uv = {M::pack2(vq[0], vq[1]), M::pack2(vq[2], vq[3])};
        *reinterpret_cast<u32x2*>(rk + 16 * ds + 4 * g) = uk;
        *reinterpret_cast<u32x2*>(rv + 16 * ds + 4 * g) = uv;
      }
    }
  }
}

bool attn_mfma_supported(int D) { return D == 64 || D == 128; }

template <typename T> int attn_fwd_mfma(const AttnArgs& a, hipStream_t st) {
  const int64_t nb = (int64_t)((a.T + FBM - 1) / FBM) * a.B * a.H;
  if (nb > 0x7fffffffLL) return KAT_EUNSUPPORTED;
  dim3 grid((unsigned)nb);
  if (a.D == 128)
    hipLaunchKernelGGL((attn_fwd_mfma_k<T, 128>), grid, dim3(256), 0, st, a);
  else if (a.D == 64)
    hipLaunchKernelGGL((attn_fwd_mfma_k<T, 64>), grid, dim3(256), 0, st, a);
  else
    return KAT_EUNSUPPORTED;
  return check_launch("kat_attn_fwd (mfma)");
}

template <typename T>
int attn_bwd_mfma(const AttnArgs& a, const float* delta, const float* cinv, hipStream_t st) {
  const int64_t nk = (int64_t)((a.T + KBN - 1) / KBN) * a.B * a.H;
  const int64_t nq = (int64_t)((a.T + FBM - 1) / FBM) * a.B * a.H;
  if (nk > 0x7fffffffLL || nq > 0x7fffffffLL) return KAT_EUNSUPPORTED;
  dim3 gk((unsigned)nk), gq((unsigned)nq);
  if (a.D == 128) {
    hipLaunchKernelGGL((attn_bwd_dkv_mfma_k<T, 128>), gk, dim3(256), 0, st, a, delta, cinv);
    if (int rc = check_launch("kat_attn_bwd (dkv, mfma)")) return rc;
    hipLaunchKernelGGL((attn_bwd_dq_mfma_k<T, 128>), gq, dim3(256), 0, st, a, delta, cinv);
  } else if (a.D == 64) {
    hipLaunchKernelGGL((attn_bwd_dkv_mfma_k<T, 64>), gk, dim3(256), 0, st, a, delta, cinv);
    if (int rc = check_launch("kat_attn_bwd (dkv, mfma)")) return rc;
    hipLaunchKernelGGL((attn_bwd_dq_mfma_k<T, 64>), gq, dim3(256), 0, st, a, delta, cinv);
  } else {
    return KAT_EUNSUPPORTED;
  }
  return check_launch("kat_attn_bwd (dq, mfma)");
}

template int attn_fwd_mfma<bf16>(const AttnArgs&, hipStream_t);
template int attn_fwd_mfma<f16>(const AttnArgs&, hipStream_t);
template int attn_bwd_mfma<bf16>(const AttnArgs&, const float*, const float*, hipStream_t);
template int attn_bwd_mfma<f16>(const AttnArgs&, const float*, const float*, hipStream_t);

}  // namespace kat
