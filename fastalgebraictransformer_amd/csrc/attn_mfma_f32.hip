// fp32 rational attention (forward and backward) on gfx950 matrix cores:
// v_mfma_f32_16x16x4_f32.
//
// The fp32 form of the MFMA forward (attn_mfma_kernels.h): the same math
// (forward.py:110-159: s = scale q.k - slope (i - j), f = sigma(s)^4 = t^4 / 16
// with t = 1 + s / (|s| + 1), no running maximum, o = sum f v / (L + eps)), with
// fp32 operands, products and sums throughout -- the precision of the
// reference's fp32 kernel, which loads every operand .to(tl.float32)
// (forward.py:103,126,146) -- on the fp32 matrix instruction instead of the
// VALU (the tiled kernels in attn_generic.hip: ~3 TFLOP/s at config 1).
//
// Block: 4 waves of 16 queries (64 queries; small problems such as config 1,
// B=2, H=12, S=512, still give 192 blocks). K and V stream through LDS in
// tiles of KT keys (64; 32 at D = 128, 16 at D = 256), double-buffered
// LDS-DMA. Per 16-key
// group of a tile a wave computes
//   S^T[key][q] = K Q^T      A = K (LDS, one ds_read_b128 per 4 k-steps)
//                            B = Q^T (VGPRs for the whole kernel)
//   f = t^4 of S^T (the C layout: lane (g, li) holds keys 4 g + j, query li)
//   O^T[d][q] += V^T f^T     A = V^T (LDS, ds_read_b32)  B = f itself: the
//                            k-index of the 16x16x4 product is the lane group
//                            g, and lane (g, li) holds key 4 g + j in step j,
//                            so S^T's C registers are O^T's B operand as they
//                            stand (no conversion, no shuffle).
// In QK^T the k-steps take the head dim in the order d = 16 m + 4 g + j
// (block m, step j, lane group g): a lane's four steps of block m read 16
// contiguous bytes of its key row, and its Q fragment is the float4 at the same
// columns of its query row.
// LDS tiles reuse the 16-bit tile helpers of attn_mfma_dev.h with rows of 2 D
// 16-bit units (the same swizzle: the row reads above are those of the bf16
// kernels' A fragments, and the four rows 4 g + j of a V read land in four
// different bank groups).

#include <algorithm>

#include "attn_common.h"
#include "attn_mfma_dev.h"
#include "kat_internal.h"

namespace kat {

using namespace mfma;

namespace {

constexpr int kF32W = 4;                // waves per block
constexpr int kF32Q = 16;               // queries per wave
constexpr int kF32BM = kF32W * kF32Q;   // queries per block
constexpr int kModeCausalF = 1;
constexpr int kModeKeyMaskF = 2;
template <int D> constexpr int f32_kt() { return D >= 256 ? 16 : D >= 128 ? 32 : 64; }  // keys per LDS tile

__device__ __forceinline__ f32x4 mma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Schedule of a loop over M d blocks that each take NR LDS reads and NM
// MFMAs on them: the reads run one block ahead of the MFMAs (0x100: LDS reads,
// 0x008: MFMA), and nothing moves across the call (reads hoisted further keep
// too many values live: spills at D >= 128).
template <int M, int NR, int NM> __device__ __forceinline__ void f32_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
  for (int m = 0; m < M - 1; ++m) {
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
  __builtin_amdgcn_sched_barrier(0);
}

// D = 256: one block per CU (one wave per SIMD, 512 registers: the Q fragments
// and O accumulators take 128)
template <int D, int MODE>
__global__ __launch_bounds__(64 * kF32W, D >= 256 ? 1 : 2) void attn_fwd_f32_k(AttnArgs a) {
  constexpr int D16 = 2 * D;  // a row in 16-bit units, the unit of the tile helpers
  constexpr int KT = f32_kt<D>();
  constexpr int M = D / 16;  // 16-column blocks of d: 4 k-steps of QK^T each; O^T subtiles
  constexpr bool kCausal = (MODE & kModeCausalF) != 0;
  constexpr bool kKM = (MODE & kModeKeyMaskF) != 0;
  constexpr uint64_t kAll = KT == 64 ? ~0ull : (1ull << KT) - 1ull;  // every key of a tile valid
  __shared__ short sk[2][KT * D16];
  __shared__ short sv[2][KT * D16];

  const int T_ = a.T, H = a.H;
  int bh, rank;
  block_order((int)blockIdx.x, a.B * H, bh, rank);
  const int n_qt = (T_ + kF32BM - 1) / kF32BM;
  const int q0 = (n_qt - 1 - rank) * kF32BM;
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qw = q0 + kF32Q * w;

  const float* qp = (const float*)a.q + b * a.sq[0] + h * a.sq[1];
  const float* kp = (const float*)a.k + b * a.sk[0] + h * a.sk[1];
  const float* vp = (const float*)a.v + b * a.sv[0] + h * a.sv[1];
  const int DR = a.D;  // the head dim (<= D; columns DR .. D - 1 read as zeros)
  const uint32_t sq2 = (uint32_t)a.sq[2], sk2 = (uint32_t)a.sk[2], sv2 = (uint32_t)a.sv[2];
  // extents and strides in 16-bit units for the tile helpers
  const uint32_t kbytes = row_bytes(T_, 2 * sk2, 2 * DR), vbytes = row_bytes(T_, 2 * sv2, 2 * DR);
  const float slope = a.slopes[h];
  const float scale = a.scale;

  // Q^T fragments: lane (g, li) holds Q[qw + li][16 m + 4 g .. + 3] (step j of block m: element j)
  f32x4 qf[M];
  {
    const __amdgpu_buffer_rsrc_t rq = rsrc(qp, row_bytes(T_, 2 * sq2, 2 * DR));
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int col = 16 * m + 4 * g;
      qf[m] = __builtin_bit_cast(f32x4, load16(rq, col_off(((uint32_t)(qw + li) * sq2 + col) * 4, col, DR)));
    }
  }
  // element j of a 16-key group starting at key kh: key = kh + 4 g + j, query
  // qw + li, bias -slope |key - q| (forward.py:129-133) from the exact integer
  // distance kh - qw + dlo[j]; added after the product (a bias carried in the
  // accumulator would set the rounding of every partial sum)
  int dlo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) dlo[j] = 4 * g + j - li;
  const float nslope = -slope;
  uint64_t vm = ~0ull;  // key validity of the current tile (bit r: key kcur + r)
  int kcur = 0;
  const uint8_t* kmb = kKM ? a.km + (int64_t)b * a.skm : nullptr;

  f32x4 oacc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) oacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;

  TileDma<D16, kF32W, KT> dk, dv;
  dk.init(w, lane, 2 * sk2, 2 * DR);
  dv.init(w, lane, 2 * sv2, 2 * DR);

  // one 16-key group at tile row hr (key kh): S^T, its f, and O^T += V^T f^T
  auto group = [&](auto masked_tag, int hr, int kh, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool kVM = kKM || !kCausal;
    f32x4 s_ = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const f32x4 kf = *reinterpret_cast<const f32x4*>(ks_ + soff<D16>(hr + li, 32 * m + 8 * g));
#pragma unroll
      for (int j = 0; j < 4; ++j) s_ = mma_f32(kf[j], qf[m][j], s_);
    }
    f32_interleave<M, 1, 4>();
    uint32_t nib = 0;
    if constexpr (MASKED && kVM) nib = (uint32_t)(vm >> (kh - kcur + 4 * g));
    const int kq = kh - qw;
    float f[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = fmaf(s_[j], scale, nslope * (float)abs(kq + dlo[j]));
      const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
      const float t = fmaf(s, r, 1.f);
      const float t2 = t * t;
      f[j] = t2 * t2;
      if (MASKED && kCausal && kh + 4 * g + j > qw + li) f[j] = 0.f;
      if (MASKED && kVM && !((nib >> j) & 1u)) f[j] = 0.f;
    }
    lsum += (f[0] + f[1]) + (f[2] + f[3]);
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float vv = *reinterpret_cast<const float*>(vs_ + soff<D16>(hr + 4 * g + j, 32 * m + 2 * li));
        oacc[m] = mma_f32(vv, f[j], oacc[m]);
      }
    f32_interleave<M, 4, 4>();
  };
  auto tile = [&](auto masked_tag, int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
#pragma unroll
    for (int hr = 0; hr < KT; hr += 16) group(masked_tag, hr, k0 + hr, ks_, vs_);
  };
  // which variant a tile takes (as in the bf16 forward): causal without a
  // padding mask -- below the diagonal plain, straddling it masked, above it
  // skipped; otherwise a tile wholly on one side of the diagonal with every
  // key valid is plain, one with no valid key skipped, any other masked
  auto tile_step = [&](int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    if constexpr (kCausal && !kKM) {
      if (k0 + KT - 1 <= qw)
        tile(std::false_type{}, k0, ks_, vs_);
      else if (k0 <= qw + kF32Q - 1)
        tile(std::true_type{}, k0, ks_, vs_);
    } else {
      // (the bias -slope |key - q| needs no per-score handling off the diagonal)
      const bool plain = (!kCausal || k0 + KT - 1 <= qw) && vm == kAll;
      if (vm == 0ull || (kCausal && k0 > qw + kF32Q - 1)) {
      } else if (plain) {
        tile(std::false_type{}, k0, ks_, vs_);
      } else {
        tile(std::true_type{}, k0, ks_, vs_);
      }
    }
  };

  const int n_kt = kCausal ? (std::min(q0 + kF32BM, T_) + KT - 1) / KT : (T_ + KT - 1) / KT;
  // this lane's padding-mask byte of key tile kt (0 past the tile or the end)
  auto kmbyte = [&](int kt) __attribute__((always_inline)) {
    const int j = kt * KT + lane;
    return (kKM && lane < KT && j < T_) ? (uint32_t)kmb[j] : 0u;
  };
  uint32_t kmn = kmbyte(0);
  dk.issue(sk[0], kp, kbytes, 0, 2 * sk2, w);
  dv.issue(sv[0], vp, vbytes, 0, 2 * sv2, w);
  dma_wait();
  __syncthreads();
  auto step = [&](int kt, auto buf_tag) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_tag)::value;
    if (kt + 1 < n_kt) {
      dk.issue(sk[buf ^ 1], kp, kbytes, (kt + 1) * KT, 2 * sk2, w);
      dv.issue(sv[buf ^ 1], vp, vbytes, (kt + 1) * KT, 2 * sv2, w);
    }
    const int k0 = kt * KT;
    kcur = k0;
    if constexpr (kKM) {
      vm = __builtin_amdgcn_ballot_w64(kmn != 0u);
      if (kt + 1 < n_kt) kmn = kmbyte(kt + 1);
    } else if constexpr (!kCausal) {
      vm = T_ - k0 >= KT ? kAll : (1ull << (T_ - k0)) - 1ull;
    }
    tile_step(k0, sk[buf], sv[buf]);
    dma_wait();
    __syncthreads();
  };
  for (int kt = 0; kt < n_kt; kt += 2) {
    step(kt, std::integral_constant<int, 0>{});
    if (kt + 1 < n_kt) step(kt + 1, std::integral_constant<int, 1>{});
  }

  // epilogue: L' across the 4 lane groups; lane (g, li) holds O^T[16 m + 4 g + jj][li]
  float l = lsum;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const int qrow = qw + li;
  if (qrow >= T_) return;
  const float inv = 1.f / (l + 16.f * a.eps);
  float* __restrict__ Lp = a.L + b * a.sl[0] + h * a.sl[1];
  if (g == 0) Lp[(int64_t)qrow * a.sl[2]] = l * 0.0625f;
  float* __restrict__ op = (float*)a.o + b * a.so[0] + h * a.so[1] + (int64_t)qrow * a.so[2];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int col = 16 * m + 4 * g;
    if (col < DR) *reinterpret_cast<f32x4*>(op + col) = oacc[m] * inv;
  }
}

// ============================================================================
// Backward, recomputing S and dP from the inputs (no stored tiles), with p, g
// and dS as the reference forms them (backward.py:128-151, 232-260):
//   p = sigma^4 / (L + eps),  g = 2 / ((|s| + 1)^2 (sigma + eps)),
//   dS = p g (dP - Delta),  dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO;
// with t = 2 sigma = 1 + s r, r = 1 / (|s| + 1) and cinv = 1 / (16 (L + eps)):
// p = t^4 cinv and g = 4 r^2 / (t + 2 eps).
//   bwd_dq_f32   query blocks as in the forward: S^T = K Q^T and
//                dP^T = V dO^T (A = K, V rows; B = Q^T, dO^T in VGPRs),
//                dS^T, dQ^T += K^T dS^T (A = K read by columns, B = dS^T
//                in its C registers as they stand)
//   bwd_dkv_f32  key blocks, 16 keys per wave: S = Q K^T, dP = dO V^T
//                (A = Q, dO rows; B = K^T, V^T in VGPRs), P and dS,
//                dV^T += dO^T P, dK^T += Q^T dS (A = dO, Q read by
//                columns; B = P, dS as they stand)
// Both run as the blocks of one launch, attn_bwd_f32_k. Delta and cinv come
// from attn_delta (the tiled path's first pass).
// ============================================================================
constexpr int kF32KB = kF32W * 16;  // keys per dK/dV block
template <int D> constexpr int f32_qt() { return D >= 256 ? 16 : D >= 128 ? 32 : 64; }  // queries per LDS tile

// p and dS of one score (s: the biased, scaled score)
__device__ __forceinline__ void p_ds(float s, float dp, float ci, float dl, float eps2, float& p, float& ds) {
  const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
  const float t = fmaf(s, r, 1.f);
  const float t2 = t * t;
  p = t2 * t2 * ci;
  ds = p * (4.f * r * r * __builtin_amdgcn_rcpf(t + eps2)) * (dp - dl);
}

// the LDS of the dQ and of the dK/dV blocks, which share one launch
template <int D> struct F32DqSmem {
  short k[2][f32_kt<D>() * 2 * D];
  short v[2][f32_kt<D>() * 2 * D];
};
template <int D> struct F32DkvSmem {
  short q[2][f32_qt<D>() * 2 * D];
  short g[2][f32_qt<D>() * 2 * D];
  float st[2][2][f32_qt<D>()];  // per tile: cinv, then Delta, of its queries
};
template <int D> union F32BwdSmem {
  F32DqSmem<D> dq;
  F32DkvSmem<D> dkv;
};

// bid: the block's index among the dQ blocks
template <int D, int MODE>
__device__ __forceinline__ void bwd_dq_f32(const AttnArgs& a, const float* __restrict__ delta,
                                           const float* __restrict__ cinv, int bid, F32DqSmem<D>& sm) {
  constexpr int D16 = 2 * D;
  constexpr int KT = f32_kt<D>();
  constexpr int M = D / 16;
  constexpr bool kCausal = (MODE & kModeCausalF) != 0;
  constexpr bool kKM = (MODE & kModeKeyMaskF) != 0;
  constexpr uint64_t kAll = KT == 64 ? ~0ull : (1ull << KT) - 1ull;
  short (&sk)[2][KT * D16] = sm.k;
  short (&sv)[2][KT * D16] = sm.v;

  const int T_ = a.T, H = a.H;
  int bh, rank;
  block_order(bid, a.B * H, bh, rank);
  const int n_qt = (T_ + kF32BM - 1) / kF32BM;
  const int q0 = (n_qt - 1 - rank) * kF32BM;
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qw = q0 + kF32Q * w;

  const float* qp = (const float*)a.q + b * a.sq[0] + h * a.sq[1];
  const float* kp = (const float*)a.k + b * a.sk[0] + h * a.sk[1];
  const float* vp = (const float*)a.v + b * a.sv[0] + h * a.sv[1];
  const float* gp = (const float*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const int DR = a.D;
  const uint32_t sq2 = (uint32_t)a.sq[2], sk2 = (uint32_t)a.sk[2], sv2 = (uint32_t)a.sv[2];
  const uint32_t sg2 = (uint32_t)a.sdo[2];
  const uint32_t kbytes = row_bytes(T_, 2 * sk2, 2 * DR), vbytes = row_bytes(T_, 2 * sv2, 2 * DR);
  const float slope = a.slopes[h];
  const float scale = a.scale;
  const float eps2 = 2.f * a.eps;

  // Q^T and dO^T fragments: lane (g, li) holds row qw + li, columns 16 m + 4 g .. + 3
  f32x4 qf[M], gf[M];
  {
    const __amdgpu_buffer_rsrc_t rq = rsrc(qp, row_bytes(T_, 2 * sq2, 2 * DR));
    const __amdgpu_buffer_rsrc_t rg = rsrc(gp, row_bytes(T_, 2 * sg2, 2 * DR));
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int col = 16 * m + 4 * g;
      qf[m] = __builtin_bit_cast(f32x4, load16(rq, col_off(((uint32_t)(qw + li) * sq2 + col) * 4, col, DR)));
      gf[m] = __builtin_bit_cast(f32x4, load16(rg, col_off(((uint32_t)(qw + li) * sg2 + col) * 4, col, DR)));
    }
  }
  const int qrow = qw + li;
  const bool qin = qrow < T_;
  const float ci = qin ? cinv[(int64_t)bh * T_ + qrow] : 0.f;  // rows past T: p = dS = 0
  const float dl = qin ? delta[(int64_t)bh * T_ + qrow] : 0.f;
  int dlo[4];  // as in the forward: bias -slope |kh - qw + dlo[j]|
#pragma unroll
  for (int j = 0; j < 4; ++j) dlo[j] = 4 * g + j - li;
  const float nslope = -slope;
  uint64_t vm = ~0ull;
  int kcur = 0;
  const uint8_t* kmb = kKM ? a.km + (int64_t)b * a.skm : nullptr;

  f32x4 qacc[M];  // dQ^T: lane (g, li) holds [16 m + 4 g + jj][query li]
#pragma unroll
  for (int m = 0; m < M; ++m) qacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

  TileDma<D16, kF32W, KT> dk, dv;
  dk.init(w, lane, 2 * sk2, 2 * DR);
  dv.init(w, lane, 2 * sv2, 2 * DR);

  auto group = [&](auto masked_tag, int hr, int kh, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool kVM = kKM || !kCausal;
    f32x4 s_ = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const f32x4 kf = *reinterpret_cast<const f32x4*>(ks_ + soff<D16>(hr + li, 32 * m + 8 * g));
      const f32x4 vf = *reinterpret_cast<const f32x4*>(vs_ + soff<D16>(hr + li, 32 * m + 8 * g));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s_ = mma_f32(kf[j], qf[m][j], s_);
        dp = mma_f32(vf[j], gf[m][j], dp);
      }
    }
    f32_interleave<M, 2, 8>();
    uint32_t nib = 0;
    if constexpr (MASKED && kVM) nib = (uint32_t)(vm >> (kh - kcur + 4 * g));
    const int kq = kh - qw;
    float dsv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = fmaf(s_[j], scale, nslope * (float)abs(kq + dlo[j]));
      float p;
      p_ds(s, dp[j], ci, dl, eps2, p, dsv[j]);
      if (MASKED && kCausal && kh + 4 * g + j > qrow) dsv[j] = 0.f;
      if (MASKED && kVM && !((nib >> j) & 1u)) dsv[j] = 0.f;
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float kv = *reinterpret_cast<const float*>(ks_ + soff<D16>(hr + 4 * g + j, 32 * m + 2 * li));
        qacc[m] = mma_f32(kv, dsv[j], qacc[m]);
      }
    f32_interleave<M, 4, 4>();
  };
  auto tile = [&](auto masked_tag, int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
#pragma unroll
    for (int hr = 0; hr < KT; hr += 16) group(masked_tag, hr, k0 + hr, ks_, vs_);
  };
  auto tile_step = [&](int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    if constexpr (kCausal && !kKM) {
      if (k0 + KT - 1 <= qw)
        tile(std::false_type{}, k0, ks_, vs_);
      else if (k0 <= qw + kF32Q - 1)
        tile(std::true_type{}, k0, ks_, vs_);
    } else {
      // (the bias -slope |key - q| needs no per-score handling off the diagonal)
      const bool plain = (!kCausal || k0 + KT - 1 <= qw) && vm == kAll;
      if (vm == 0ull || (kCausal && k0 > qw + kF32Q - 1)) {
      } else if (plain) {
        tile(std::false_type{}, k0, ks_, vs_);
      } else {
        tile(std::true_type{}, k0, ks_, vs_);
      }
    }
  };

  const int n_kt = kCausal ? (std::min(q0 + kF32BM, T_) + KT - 1) / KT : (T_ + KT - 1) / KT;
  auto kmbyte = [&](int kt) __attribute__((always_inline)) {
    const int j = kt * KT + lane;
    return (kKM && lane < KT && j < T_) ? (uint32_t)kmb[j] : 0u;
  };
  uint32_t kmn = kmbyte(0);
  dk.issue(sk[0], kp, kbytes, 0, 2 * sk2, w);
  dv.issue(sv[0], vp, vbytes, 0, 2 * sv2, w);
  dma_wait();
  __syncthreads();
  auto step = [&](int kt, auto buf_tag) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_tag)::value;
    if (kt + 1 < n_kt) {
      dk.issue(sk[buf ^ 1], kp, kbytes, (kt + 1) * KT, 2 * sk2, w);
      dv.issue(sv[buf ^ 1], vp, vbytes, (kt + 1) * KT, 2 * sv2, w);
    }
    const int k0 = kt * KT;
    kcur = k0;
    if constexpr (kKM) {
      vm = __builtin_amdgcn_ballot_w64(kmn != 0u);
      if (kt + 1 < n_kt) kmn = kmbyte(kt + 1);
    } else if constexpr (!kCausal) {
      vm = T_ - k0 >= KT ? kAll : (1ull << (T_ - k0)) - 1ull;
    }
    tile_step(k0, sk[buf], sv[buf]);
    dma_wait();
    __syncthreads();
  };
  for (int kt = 0; kt < n_kt; kt += 2) {
    step(kt, std::integral_constant<int, 0>{});
    if (kt + 1 < n_kt) step(kt + 1, std::integral_constant<int, 1>{});
  }
  if (!qin) return;
  float* __restrict__ dqp = (float*)a.dq + b * a.sdq[0] + h * a.sdq[1] + (int64_t)qrow * a.sdq[2];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int col = 16 * m + 4 * g;
    if (col < DR) *reinterpret_cast<f32x4*>(dqp + col) = qacc[m] * scale;
  }
}

// D = 256: the K^T and V^T fragments and the dV^T and dK^T accumulators alone
// take 256 VGPRs, so one block per CU (one wave per SIMD, 512 registers)
// bid: the block's index among the dK/dV blocks
template <int D, int MODE>
__device__ __forceinline__ void bwd_dkv_f32(const AttnArgs& a, const float* __restrict__ delta,
                                            const float* __restrict__ cinv, int bid, F32DkvSmem<D>& sm) {
  constexpr int D16 = 2 * D;
  constexpr int QT = f32_qt<D>();
  constexpr int M = D / 16;
  constexpr bool kCausal = (MODE & kModeCausalF) != 0;
  constexpr bool kKM = (MODE & kModeKeyMaskF) != 0;
  short (&sq)[2][QT * D16] = sm.q;
  short (&sg)[2][QT * D16] = sm.g;
  float (&sst)[2][2][QT] = sm.st;

  const int T_ = a.T, H = a.H;
  int bh, rank;
  block_order(bid, a.B * H, bh, rank);  // rank 0: the first keys (most queries)
  const int k0 = rank * kF32KB;
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int kw = k0 + 16 * w;  // this wave's 16 keys
  const int key = kw + li;     // lane (g, li): key li of the wave, queries 4 g + jj of a group

  const float* qp = (const float*)a.q + b * a.sq[0] + h * a.sq[1];
  const float* kp = (const float*)a.k + b * a.sk[0] + h * a.sk[1];
  const float* vp = (const float*)a.v + b * a.sv[0] + h * a.sv[1];
  const float* gp = (const float*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const int DR = a.D;
  const uint32_t sq2 = (uint32_t)a.sq[2], sk2 = (uint32_t)a.sk[2], sv2 = (uint32_t)a.sv[2];
  const uint32_t sg2 = (uint32_t)a.sdo[2];
  const uint32_t qbytes = row_bytes(T_, 2 * sq2, 2 * DR), gbytes = row_bytes(T_, 2 * sg2, 2 * DR);
  const float slope = a.slopes[h];
  const float scale = a.scale;
  const float eps2 = 2.f * a.eps;
  const float* cinv_h = cinv + (int64_t)bh * T_;
  const float* delta_h = delta + (int64_t)bh * T_;

  // K^T and V^T fragments: lane (g, li) holds row `key`, columns 16 m + 4 g .. + 3
  f32x4 kf[M], vf[M];
  {
    const __amdgpu_buffer_rsrc_t rk = rsrc(kp, row_bytes(T_, 2 * sk2, 2 * DR));
    const __amdgpu_buffer_rsrc_t rv = rsrc(vp, row_bytes(T_, 2 * sv2, 2 * DR));
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int col = 16 * m + 4 * g;
      kf[m] = __builtin_bit_cast(f32x4, load16(rk, col_off(((uint32_t)key * sk2 + col) * 4, col, DR)));
      vf[m] = __builtin_bit_cast(f32x4, load16(rv, col_off(((uint32_t)key * sv2 + col) * 4, col, DR)));
    }
  }
  // S layout: lane (g, li) element jj holds query qh + 4 g + jj, key `key`;
  // bias -slope |key - q| from the exact integer distance kw - qh + dlo[jj]
  int dlo[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) dlo[jj] = li - 4 * g - jj;
  const float nslope = -slope;

  f32x4 vacc[M], kacc[M];  // dV^T, dK^T: lane (g, li) holds [16 m + 4 g + jj][key li]
#pragma unroll
  for (int m = 0; m < M; ++m) {
    vacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    kacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  TileDma<D16, kF32W, QT> dq_, dg_;
  dq_.init(w, lane, 2 * sq2, 2 * DR);
  dg_.init(w, lane, 2 * sg2, 2 * DR);

  // one 16-query group at tile row hr (query qh); causal: scores with the key
  // after the query masked per score (the MFMAs dominate this kernel, so one
  // variant serves every group: fewer live registers than one per side of the
  // diagonal)
  auto group = [&](int hr, int qh, const short* qs_, const short* gs_, const float* st_) __attribute__((always_inline)) {
    f32x4 s_ = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const f32x4 qa = *reinterpret_cast<const f32x4*>(qs_ + soff<D16>(hr + li, 32 * m + 8 * g));
      const f32x4 ga = *reinterpret_cast<const f32x4*>(gs_ + soff<D16>(hr + li, 32 * m + 8 * g));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s_ = mma_f32(qa[j], kf[m][j], s_);
        dp = mma_f32(ga[j], vf[m][j], dp);
      }
    }
    f32_interleave<M, 2, 8>();
    const f32x4 c4v = *reinterpret_cast<const f32x4*>(st_ + hr + 4 * g);
    const f32x4 dlv = *reinterpret_cast<const f32x4*>(st_ + QT + hr + 4 * g);
    const int kq = kw - qh;
    float pv[4], dsv[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int dq = kq + dlo[jj];  // key - query; > 0: the key lies after the query
      const float s = fmaf(s_[jj], scale, nslope * (float)abs(dq));
      p_ds(s, dp[jj], c4v[jj], dlv[jj], eps2, pv[jj], dsv[jj]);
      if (kCausal && dq > 0) {
        pv[jj] = 0.f;
        dsv[jj] = 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int off = soff<D16>(hr + 4 * g + j, 32 * m + 2 * li);
        vacc[m] = mma_f32(*reinterpret_cast<const float*>(gs_ + off), pv[j], vacc[m]);
        kacc[m] = mma_f32(*reinterpret_cast<const float*>(qs_ + off), dsv[j], kacc[m]);
      }
    f32_interleave<M, 8, 8>();
  };
  // a query tile: its 16-query groups (causal: those with a query at or
  // after one of the wave's keys)
  auto tile = [&](int q0t, const short* qs_, const short* gs_, const float* st_) __attribute__((always_inline)) {
#pragma unroll
    for (int hr = 0; hr < QT; hr += 16) {
      const int qh = q0t + hr;
      if (!kCausal || qh + 15 >= kw) group(hr, qh, qs_, gs_, st_);
    }
  };

  // query tiles: causal, from the tile holding k0 on; otherwise all
  const int qt0 = kCausal ? k0 / QT : 0;
  const int n_qt = (T_ + QT - 1) / QT;
  // the stats of a tile's queries (0 past T: p = dS = 0 there), staged
  // through a register: threads 0 .. QT - 1 cinv, QT .. 2 QT - 1 Delta
  auto stat = [&](int qt) __attribute__((always_inline)) {
    const int qq = qt * QT + (tid % QT);
    if (tid >= 2 * QT || qq >= T_) return 0.f;
    return tid < QT ? cinv_h[qq] : delta_h[qq];
  };
  if (qt0 < n_qt) {
    dq_.issue(sq[0], qp, qbytes, qt0 * QT, 2 * sq2, w);
    dg_.issue(sg[0], gp, gbytes, qt0 * QT, 2 * sg2, w);
    if (tid < 2 * QT) sst[0][tid / QT][tid % QT] = stat(qt0);
  }
  dma_wait();
  __syncthreads();
  auto step = [&](int qt, auto buf_tag) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_tag)::value;
    float stn = 0.f;
    if (qt + 1 < n_qt) {
      dq_.issue(sq[buf ^ 1], qp, qbytes, (qt + 1) * QT, 2 * sq2, w);
      dg_.issue(sg[buf ^ 1], gp, gbytes, (qt + 1) * QT, 2 * sg2, w);
      stn = stat(qt + 1);
    }
    tile(qt * QT, sq[buf], sg[buf], &sst[buf][0][0]);
    if (qt + 1 < n_qt && tid < 2 * QT) sst[buf ^ 1][tid / QT][tid % QT] = stn;
    dma_wait();
    __syncthreads();
  };
  for (int qt = qt0; qt < n_qt; qt += 2) {
    step(qt, std::integral_constant<int, 0>{});
    if (qt + 1 < n_qt) step(qt + 1, std::integral_constant<int, 1>{});
  }

  if (key >= T_) return;
  const bool kin = !kKM || a.km[(int64_t)b * a.skm + key] != 0;  // a dropped key's gradients are 0
  float* __restrict__ dvp = (float*)a.dv + b * a.sdv[0] + h * a.sdv[1] + (int64_t)key * a.sdv[2];
  float* __restrict__ dkp = (float*)a.dk + b * a.sdk[0] + h * a.sdk[1] + (int64_t)key * a.sdk[2];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int col = 16 * m + 4 * g;
    if (col < DR) {
      *reinterpret_cast<f32x4*>(dvp + col) = kin ? vacc[m] : f32x4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4*>(dkp + col) = kin ? kacc[m] * scale : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
}

// The backward's dK/dV and dQ blocks in one launch (they are independent: both
// take Delta and cinv from attn_delta): blocks [0, nk) run dK/dV, blocks
// [nkp, nkp + nq) dQ, nkp = nk rounded up to a multiple of 8 (the blocks in
// between exit at once) so that each part's block ids keep their XCD (id % 8)
// for block_order. Small problems run both parts side by side (config 1,
// B=2, H=12, S=512: 192 + 192 blocks on 256 CUs) instead of one after the
// other; the LDS of the two parts is shared, registers are the larger part's.
template <int D, int MODE>
__global__ __launch_bounds__(64 * kF32W, D >= 256 ? 1 : 2) void attn_bwd_f32_k(AttnArgs a, const float* __restrict__ delta,
                                                              const float* __restrict__ cinv, int nk, int nkp) {
  __shared__ F32BwdSmem<D> sm;
  const int id = (int)blockIdx.x;
  if (id < nk)
    bwd_dkv_f32<D, MODE>(a, delta, cinv, id, sm.dkv);
  else if (id >= nkp)
    bwd_dq_f32<D, MODE>(a, delta, cinv, id - nkp, sm.dq);
}

// layout widths of the fp32 kernels: 32, 64, 128, 256 (a head dim between
// them, a multiple of 4, runs in the next width with its columns past D as zeros)
int f32_width(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }

#define KAT_F32_MODE_SWITCH(a, ...)                                                     \
  switch ((a.causal ? kModeCausalF : 0) | (a.km != nullptr ? kModeKeyMaskF : 0)) {      \
    case kModeCausalF: { constexpr int MODE = kModeCausalF; __VA_ARGS__; }              \
    case kModeCausalF | kModeKeyMaskF: { constexpr int MODE = kModeCausalF | kModeKeyMaskF; __VA_ARGS__; } \
    case kModeKeyMaskF: { constexpr int MODE = kModeKeyMaskF; __VA_ARGS__; }            \
    default: { constexpr int MODE = 0; __VA_ARGS__; }                                   \
  }

template <int D, int MODE> int launch_fwd_f32(const AttnArgs& a, hipStream_t st) {
  const int64_t nb = (int64_t)((a.T + kF32BM - 1) / kF32BM) * a.B * a.H;
  hipLaunchKernelGGL((attn_fwd_f32_k<D, MODE>), dim3((unsigned)nb), dim3(64 * kF32W), 0, st, a);
  return check_launch("kat_attn_fwd (fp32 mfma)");
}

template <int D, int MODE>
int launch_bwd_f32(const AttnArgs& a, const float* delta, const float* cinv, hipStream_t st) {
  const int64_t nq = (int64_t)((a.T + kF32BM - 1) / kF32BM) * a.B * a.H;
  const int64_t nk = (int64_t)((a.T + kF32KB - 1) / kF32KB) * a.B * a.H;
  const int64_t nkp = (nk + 7) & ~(int64_t)7;
  hipLaunchKernelGGL((attn_bwd_f32_k<D, MODE>), dim3((unsigned)(nkp + nq)), dim3(64 * kF32W), 0, st, a, delta,
                     cinv, (int)nk, (int)nkp);
  return check_launch("kat_attn_bwd (fp32 mfma)");
}

// 31-bit byte offsets per (b, h) slice for every row the kernels address
bool f32_offsets_ok(const AttnArgs& a, bool bwd) {
  const int64_t lim = 0x7fffffffLL;
  const int64_t* s2[4] = {&a.sq[2], &a.sk[2], &a.sv[2], &a.sdo[2]};
  for (int t = 0; t < (bwd ? 4 : 3); ++t)
    if (*s2[t] < a.D || ((int64_t)a.T + 128) * *s2[t] * 4 > lim) return false;
  // the backward's launch: dK/dV blocks (rounded up to 8) and dQ blocks
  return 2 * ((int64_t)((a.T + kF32BM - 1) / kF32BM) * a.B * a.H + 8) <= 0x7fffffffLL;
}

}  // namespace

bool attn_f32_mfma_supported(int D) { return D >= 4 && D <= 256 && D % 4 == 0; }

int attn_bwd_mfma_f32(const AttnArgs& a, const float* delta, const float* cinv, hipStream_t st) {
  if (!attn_f32_mfma_supported(a.D) || !f32_offsets_ok(a, true)) return KAT_EUNSUPPORTED;
  switch (f32_width(a.D)) {
    case 32: KAT_F32_MODE_SWITCH(a, return (launch_bwd_f32<32, MODE>(a, delta, cinv, st)));
    case 64: KAT_F32_MODE_SWITCH(a, return (launch_bwd_f32<64, MODE>(a, delta, cinv, st)));
    case 128: KAT_F32_MODE_SWITCH(a, return (launch_bwd_f32<128, MODE>(a, delta, cinv, st)));
    case 256: KAT_F32_MODE_SWITCH(a, return (launch_bwd_f32<256, MODE>(a, delta, cinv, st)));
  }
  return KAT_EUNSUPPORTED;
}

int attn_fwd_mfma_f32(const AttnArgs& a, hipStream_t st) {
  if (!attn_f32_mfma_supported(a.D) || !f32_offsets_ok(a, false)) return KAT_EUNSUPPORTED;
  switch (f32_width(a.D)) {
    case 32: KAT_F32_MODE_SWITCH(a, return (launch_fwd_f32<32, MODE>(a, st)));
    case 64: KAT_F32_MODE_SWITCH(a, return (launch_fwd_f32<64, MODE>(a, st)));
    case 128: KAT_F32_MODE_SWITCH(a, return (launch_fwd_f32<128, MODE>(a, st)));
    case 256: KAT_F32_MODE_SWITCH(a, return (launch_fwd_f32<256, MODE>(a, st)));
  }
  return KAT_EUNSUPPORTED;
}

}  // namespace kat
