// bf16 / fp16 MFMA rational attention for gfx950 (CDNA4): the kernels and
// their launchers, included by the per-width translation units
// (attn_mfma_w*.hip, which instantiate them) and by attn_mfma.hip (the C-ABI
// side: dispatch and workspace sizing).
//
// The attention math runs in three MFMA kernels, beside two streaming passes:
//   attn_fwd_k         O, L      query-tile blocks; K, V tiles stream through LDS
//   attn_bwd_prep_k    fp16 copy of Q with per-tile exponents, Delta and the
//                                row stats, the parts of the dS bounds
//   attn_bwd_stscale_k the dS exponent of each query tile; scales the row
//                                stats by it
//   attn_bwd_dkv_k     dK, dV    key-tile blocks; fp16 Q and dO tiles stream; the
//                                waves split into a dV role and a dK role; the dK
//                                role also stores the fp16 dS it computes
//   attn_bwd_dq_k      dQ        query-tile blocks: dQ = dS K over the stored dS
// Every output element is written by one wave, so results are deterministic
// (no atomics). The backward computes S, P and dS once: 5 MFMA units for the 5
// of the algorithm (S, dP, dV, dK, dQ).
//
// Common structure of the forward and dK/dV kernels (the dQ kernel is a plain
// streaming GEMM, described at it). Each wave owns 32 rows (queries, or keys
// for dK/dV; 16 or 64 keys at some head dims, see dkv_keys) whose
// operand fragments stay in VGPRs as the B operand of v_mfma_f32_16x16x32; the
// streamed side is staged 64 rows at a time by LDS-DMA into a swizzled,
// double-buffered LDS tile and read as the A operand, either row-wise
// (ds_read_b128) or transposed (ds_read_b64_tr_b16). A 64-row tile is worked in
// 16-row halves: S (and dP) for a half, the elementwise map for it, and the
// product that consumes the result once two halves (32 rows = one MFMA k-step)
// are ready; the compiler interleaves the MFMAs of one half with the VALU work
// of the previous one.
//
// Forward math (forward.py:137-159 semantics). Per score,
//   s  = scale q.k - slope (i - j),  r = 1 / (|s| + 1),  t = 1 + s r = 2 sigma(s)
//   f' = t^4 = 16 sigma^4            (no running max: sigma^4 lies in (0, 1))
//   L' = sum_j f',  o = (sum_j f' v_j) / (L' + 16 eps),  L = L' / 16.
// The factor 16 is exact in binary floating point. The ALiBi bias is split into
// a per-lane part fed to QK^T as its C input (divided by scale) and a wave-uniform
// part added by the FMA that applies the scale.
//
// Backward math. With cinv_i = 1 / (16 (L_i + eps)):
//   p  = t^4 cinv_i,   dS = p g (dP - Delta_i) = 4 cinv_i t^3 r^2 (dP - Delta_i)
//   dQ = scale dS K,   dK = scale dS^T Q,   dV = P^T dO.
// Range. dS enters the dQ and dK products in fp16 (normal range 2^-14 ..
// 65504), and so do the copies of Q and K those products (and the recomputed
// S) take. Every fp16 operand carries a power-of-two scale chosen from the
// data, and every scale is undone exactly (binary floating point):
//   * Q16 and K16: one exponent per 64-row tile of Q and per 32 keys of K
//     (tile_exp of their max |x|): 0 while max |x| lies in [2^-6, 2^15), else
//     max |x| 2^e lands in [2^14, 2^15); covered for maxima in [2^-46, 2^55].
//     Q16 is copied to HBM once (prep); K16 is formed where it is used, with
//     the same exponent in the dK/dV and dQ kernels. S comes out
//     of the MFMA scaled by both tiles' factors, which the bias and the scale
//     applied to it absorb; an accumulator is rescaled when a new tile brings
//     another exponent.
//   * dS (one copy, which both dK and dQ take): per 64-query tile, 2^kq from
//     the bound 4 cinv_i w |dP_ij - Delta_i| <= min(4.1, 1.125 4 cinv_i)
//     (||dO_i||_2 ||v_j||_2 + |Delta_i|) (w = t^3 r^2 <= 1.11, and
//     4 cinv_i w = p g <= 4 when L is the forward's row sum), maximised over
//     the tile's rows and the head's keys, so that every scaled dS stays
//     below 2^14; kq is the head's exponent unless the tile's bound lies
//     2^8 or more below the head's (then in steps of 2^8), so a dS reaches
//     fp16's subnormal range only 19 binades or more below its tile's bound.
// So the gradients are exactly equivariant under power-of-two scalings of q,
// k, v and dO, and dO's scale (a training step's is ~1e-5 .. 1e-7 per element)
// does not move dS into fp16's subnormal range.
// The reference writes g = 2 / ((|s|+1)^2 (sigma + eps)) (backward.py:145);
// these kernels use sigma in place of sigma + eps, a relative change of
// eps / (sigma + eps) in dS: <= 2e-6 wherever s >= 0, and otherwise on scores
// whose p <= (r / 2)^4 / L is itself negligible.

#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <type_traits>

#include "attn_common.h"
#include "attn_mfma_dev.h"
#include "kat_internal.h"

namespace kat {

using namespace mfma;

constexpr int kNW = 4;         // waves per block
constexpr int kRows = 32;      // rows owned per wave
constexpr int kBM = kNW * kRows;  // rows owned per block
constexpr int kBN = 64;        // streamed rows per LDS tile
// forward: 16-query subtiles per wave. 2: 32 queries per wave, two 4-wave blocks
// per CU (two waves per SIMD). 4 (64 queries per wave, one wave per SIMD, the O
// accumulators in AGPRs: 228 VGPRs + 164 AGPRs) halves the LDS and DMA traffic
// per MFMA but measured 18% slower at config 3 (0.353 vs 0.298 ms): a single
// wave issues VALU too slowly for the rational map.
constexpr int kFwdQS = 2;
constexpr int kFwdBM = kNW * 16 * kFwdQS;  // queries per forward block
// kernel modes: causal (keys j <= i) and a key padding mask; the reference's
// configuration is kModeCausal alone
constexpr int kModeCausal = 1;
constexpr int kModeKeyMask = 2;

// ============================================================================
// Forward: NW waves x 16 QS queries per block.
//   S^T[key][q]  = K Q^T (+ bias)   A = K  (LDS rows)         B = Q^T (VGPRs)
//   O^T[d][q]   += V^T P^T          A = V^T (LDS transposed)  B = P^T (from S^T)
// D <= 128: 4-wave blocks, two per CU. D = 256: the K and V tiles take 128 KB
// of LDS, so one block per CU of 8 waves (two per SIMD), 16 queries per wave
// (the Q fragments and O accumulators of 16 queries take 96 VGPRs).
// ============================================================================
template <typename T, int D, int MODE, int QS, int NW = kNW, int DE = D>
__global__ __launch_bounds__(64 * NW, NW == 4 && QS == 2 ? 2 : 1) void attn_fwd_k(AttnArgs a) {
  typedef Mfma<T> M;
  constexpr int KK = DE / 32;  // k-steps of QK^T
  constexpr int DS = DE / 16;  // 16-wide d subtiles of O^T
  constexpr bool kCausal = (MODE & kModeCausal) != 0;
  constexpr bool kKM = (MODE & kModeKeyMask) != 0;
  constexpr int RW = 16 * QS;    // queries per wave
  constexpr int BMQ = NW * RW;  // queries per block
  __shared__ short sk[2][kBN * D];
  __shared__ short sv[2][kBN * D];

  const int T_ = a.T, H = a.H;
  int bh, rank;
  block_order((int)blockIdx.x, a.B * H, bh, rank);
  const int n_qt = (T_ + BMQ - 1) / BMQ;
  const int q0 = (n_qt - 1 - rank) * BMQ;
  const int b = bh / H, h = bh - b * H;
  // the wave index stays a per-lane value here: as a scalar (wave_id) the
  // forward measured 3% slower
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qw = q0 + RW * w;

  const T* qp = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const uint32_t sq2 = (uint32_t)a.sq[2], sk2 = (uint32_t)a.sk[2], sv2 = (uint32_t)a.sv[2];
  const int DR = a.D;  // the head dim (<= D; columns DR .. D - 1 read as zeros)
  const uint32_t kbytes = row_bytes(T_, sk2, DR), vbytes = row_bytes(T_, sv2, DR);
  const float slope = a.slopes[h];
  const float scale = a.scale;

  // Q^T fragments (B operand): lane (g, li) holds Q[qw + 16 qs + li][32 kk + 8 g .. +7]
  i16x8 qf[QS][KK];
  {
    const __amdgpu_buffer_rsrc_t rq = rsrc(qp, row_bytes(T_, sq2, DR));
#pragma unroll
    for (int qs = 0; qs < QS; ++qs)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        qf[qs][kk] = load16(rq, col_off(((uint32_t)(qw + 16 * qs + li) * sq2 + 32 * kk + 8 * g) * 2,
                                        32 * kk + 8 * g, DR));
  }
  // element (qs, j) of a 16-key half starting at key kh: key = kh + 4 g + j,
  // q = qw + 16 qs + li; bias slope (key - q) = per-lane part + uniform part
  f32x4 cb;
#pragma unroll
  for (int j = 0; j < 4; ++j) cb[j] = (slope / scale) * (float)(4 * g + j - li);
  // the bias in use, sgn slope (key - q): sgn = +1 gives -slope |i - j| on and
  // below the diagonal; non-causal mode switches to sgn = -1 (negating cbx in
  // place) from the first tile wholly above it on
  f32x4 cbx = cb;
  float sgn = 1.f;
  // key validity of the current tile (bit r: key k0 + r), and its first key
  uint64_t vm = ~0ull;
  int kcur = 0;
  const uint8_t* kmb = kKM ? a.km + (int64_t)b * a.skm : nullptr;

  f32x4 oacc[DS][QS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) oacc[ds][qs] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lsum[QS];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) lsum[qs] = 0.f;

  TileDma<D, NW> dk, dv;
  dk.init(w, lane, sk2, DR);
  dv.init(w, lane, sv2, DR);

  // S^T of the 16 keys at tile rows hr .. hr + 15
  auto m1 = [&](int hr, f32x4 (&s_)[QS], const short* ks_) __attribute__((always_inline)) {
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) s_[qs] = cbx;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const i16x8 kf = lds16(ks_ + soff<D>(hr + li, 32 * kk + 8 * g));
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) s_[qs] = M::mma(kf, qf[qs][kk], s_[qs]);
    }
  };
  // f' of those scores, packed as P^T; row sums into lsum. MASKED: the
  // per-score work of a tile that straddles the diagonal or holds invalid
  // keys -- causal: keys past the query get f' = 0; non-causal: scores whose
  // bias form has the wrong sign for |i - j| are corrected; keys outside the
  // validity mask (padding mask, or past T) get f' = 0.
  auto vh = [&](auto masked_tag, int kh, const f32x4 (&s_)[QS], uint32_t (&pk)[QS][2]) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool kVM = kKM || !kCausal;  // a validity mask exists
    uint32_t nib = 0;
    if constexpr (MASKED && kVM) nib = (uint32_t)(vm >> (kh - kcur + 4 * g));
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const float tterm = (kCausal ? slope : sgn * slope) * (float)(kh - qw - 16 * qs);
      float f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float s = fmaf(s_[qs][j], scale, tterm);
        if constexpr (MASKED && !kCausal) {
          const float sd = sgn * (float)((kh + 4 * g + j) - (qw + 16 * qs + li));
          if (sd > 0.f) s = fmaf(-2.f * slope, sd, s);
        }
        const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
        const float t = fmaf(s, r, 1.f);
        const float t2 = t * t;
        f[j] = t2 * t2;
        if (MASKED && kCausal && kh + 4 * g + j > qw + 16 * qs + li) f[j] = 0.f;
        if (MASKED && kVM && !((nib >> j) & 1u)) f[j] = 0.f;
      }
      lsum[qs] += (f[0] + f[1]) + (f[2] + f[3]);
      pk[qs][0] = M::pack2(f[0], f[1]);
      pk[qs][1] = M::pack2(f[2], f[3]);
    }
  };
  // O^T += V^T P^T over the 32 keys at tile rows r0 .. r0 + 31
  auto m2 = [&](int r0, const uint32_t (&pa)[QS][2], const uint32_t (&pb)[QS][2], const short* vs_) __attribute__((always_inline)) {
    i16x8 pf[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) pf[qs] = pack_frag(pa[qs][0], pa[qs][1], pb[qs][0], pb[qs][1]);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const i16x8 vt = frag_tr<D>(vs_, r0, 16 * ds, g, li);
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) oacc[ds][qs] = M::mma(vt, pf[qs], oacc[ds][qs]);
    }
  };
  auto tile = [&](auto masked_tag, int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    f32x4 sA[QS], sB[QS];
    uint32_t pa0[QS][2], pb0[QS][2], pa1[QS][2], pb1[QS][2];
    m1(0, sA, ks_);
    m1(16, sB, ks_);
    vh(masked_tag, k0, sA, pa0);
    m1(32, sA, ks_);
    vh(masked_tag, k0 + 16, sB, pb0);
    m2(0, pa0, pb0, vs_);
    m1(48, sB, ks_);
    vh(masked_tag, k0 + 32, sA, pa1);
    vh(masked_tag, k0 + 48, sB, pb1);
    m2(32, pa1, pb1, vs_);
  };
  // which variant a tile takes. Causal without a padding mask: below the
  // diagonal plain, straddling it masked, above it skipped. Otherwise a tile
  // wholly on one side of the diagonal (causal: below it) with every key valid
  // takes the plain path, a tile with no valid key is skipped, and any other
  // tile takes the masked one; non-causal mode switches the bias sign at the
  // first tile wholly above the diagonal.
  auto tile_step = [&](int k0, const short* ks_, const short* vs_) __attribute__((always_inline)) {
    if constexpr (kCausal && !kKM) {
      if (k0 + kBN - 1 <= qw)
        tile(std::false_type{}, k0, ks_, vs_);
      else if (k0 <= qw + RW - 1)
        tile(std::true_type{}, k0, ks_, vs_);
    } else {
      bool plain;
      if constexpr (kCausal) {
        plain = k0 + kBN - 1 <= qw;
      } else {
        const bool above = k0 > qw + RW - 1;
        if (above && sgn > 0.f) {
          cbx = -cbx;
          sgn = -1.f;
        }
        plain = above || k0 + kBN - 1 <= qw;
      }
      plain = plain && vm == ~0ull;
      if (vm == 0ull || (kCausal && k0 > qw + RW - 1)) {
      } else if (plain) {
        tile(std::false_type{}, k0, ks_, vs_);
      } else {
        tile(std::true_type{}, k0, ks_, vs_);
      }
    }
  };

  const int n_kt = kCausal ? (std::min(q0 + BMQ, T_) + kBN - 1) / kBN : (T_ + kBN - 1) / kBN;
  // this lane's padding-mask byte of key tile kt (0 past the end)
  auto kmbyte = [&](int kt) __attribute__((always_inline)) {
    const int j = kt * kBN + lane;
    return (kKM && j < T_) ? (uint32_t)kmb[j] : 0u;
  };
  uint32_t kmn = kmbyte(0);  // loaded one tile ahead of its use
  dk.issue(sk[0], kp, kbytes, 0, sk2, w);
  dv.issue(sv[0], vp, vbytes, 0, sv2, w);
  dma_wait();
  __syncthreads();
  // tile kt sits in buffer kt & 1; the loop is unrolled by two so that the
  // buffer, and with it every LDS address, is a compile-time constant plus a
  // per-lane offset kept in a register
  auto step = [&](int kt, auto buf_tag) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_tag)::value;
    if (kt + 1 < n_kt) {
      dk.issue(sk[buf ^ 1], kp, kbytes, (kt + 1) * kBN, sk2, w);
      dv.issue(sv[buf ^ 1], vp, vbytes, (kt + 1) * kBN, sv2, w);
    }
    const int k0 = kt * kBN;
    kcur = k0;
    if constexpr (kKM) {
      vm = __builtin_amdgcn_ballot_w64(kmn != 0u);
      if (kt + 1 < n_kt) kmn = kmbyte(kt + 1);
    } else if constexpr (!kCausal) {
      vm = T_ - k0 >= kBN ? ~0ull : (1ull << (T_ - k0)) - 1ull;
    }
    tile_step(k0, sk[buf], sv[buf]);
    dma_wait();
    __syncthreads();
  };
  for (int kt = 0; kt < n_kt; kt += 2) {
    step(kt, std::integral_constant<int, 0>{});
    if (kt + 1 < n_kt) step(kt + 1, std::integral_constant<int, 1>{});
  }

  // epilogue: L' across the 4 lane groups, normalise; O through the wave's
  // own RW x D staging tile in the (now idle) K buffers, stored by rows
  T* __restrict__ op = (T*)a.o + b * a.so[0] + h * a.so[1];
  float* __restrict__ Lp = a.L + b * a.sl[0] + h * a.sl[1];
  static_assert(sizeof(sk) >= NW * RW * D * 2, "staging tiles fit the K buffers");
  short* const et = &sk[0][0] + w * RW * D;
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    float l = lsum[qs];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qrow = qw + 16 * qs + li;
    const float inv = 1.f / (l + 16.f * a.eps);
    if (qrow < T_ && g == 0) Lp[(int64_t)qrow * a.sl[2]] = l * 0.0625f;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const f32x4 o = oacc[ds][qs];
      epi_put(et, eoff<D>(16 * qs + li, 16 * ds + 4 * g), M::pack2(o[0] * inv, o[1] * inv),
              M::pack2(o[2] * inv, o[3] * inv));
    }
  }
  __syncthreads();  // orders the tile's writes before its reads
  epi_rows_out<T, D, RW>(et, lane, op, a.so[2], qw, T_, DR);
}

// Everything the backward's MFMA kernels take besides the inputs (the
// workspace, laid out by bwd_ws below).
struct BwdWs {
  float* stats;   // per 64-row tile [B*H][nt]: 4 cinv of its 64 rows, then -4 cinv Delta
                  // of them (two float[64]), then x 2^kq (the tile's dS exponent)
  f16* q16;       // fp16 copy of Q [B*H][T][D], scaled per 64-row tile
  int* qexp;      // per 64-row tile [B*H][nt]: its exponents
  int* kexp;      // per 32-key group [B*H][ceil(T / 32)]: the dK/dV kernel's
                  // fp16 K exponents, which the dQ kernel's K16 takes
  float* vnrm;    // per tile: max_j ||v_j||_2
  float* abnd;    // per tile: max_i c_i ||dO_i||_2    (c_i = min(4.1, 1.125 * 4 cinv_i))
  float* bbnd;    // per tile: max_i c_i |Delta_i|
  int* ktile;     // per 64-query tile [B*H][nt]: dS exponent kq
  f16* dst;       // dS^T tiles of a group of heads, or of one band of one head
  float* dqacc;   // banded calls: fp32 dQ partial sums of one head [nt][64][D]
  int group;      // heads per dK / dV + dQ launch pair (the dS^T tiles' capacity)
  int band;       // key tiles per band (nt: one band)
  size_t bytes;
};

// ============================================================================
// Backward prep, one block per 64-row tile of one (b, h). Streams the rows of
// Q, V, O and dO once:
//   q16       fp16 copy of Q scaled by 2^qexp, the tile's tile_exp of max |q|
//             (exact: a power of two; K is converted where it is used, in the
//             dK/dV and dQ kernels);
//   stats     (4 cinv_i, -4 cinv_i Delta_i), Delta_i = <dO_i, O_i>,
//             4 cinv_i = 1 / (4 (L_i + eps));
//   vnrm, abnd, bbnd  the tile's parts of the head's bound on |dS|:
//             |dS_ij| = 4 cinv_i w |dP_ij - Delta_i| with w = t^3 r^2 <= 1.11 and
//             4 cinv_i w = p g <= 4 (p <= 1 when L is the forward's row sum), and
//             |dP_ij - Delta_i| <= ||dO_i||_2 ||v_j||_2 + |Delta_i|, so
//             |dS_ij| <= abnd_t vnrm_max + bbnd_t for the rows i of tile t
//             (vnrm_max: over the head).
// A row's LPR = D / 8 lanes are consecutive lanes of one wave; the block covers
// its 64 rows in NP passes of 256 / LPR rows.
// ============================================================================
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_k(AttnArgs a, BwdWs ws) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int NP = 64 / RPP;
  __shared__ float red[4][4];
  const int nt = (a.T + 63) / 64;
  const int bh = (int)(blockIdx.x / (unsigned)nt), t = (int)blockIdx.x - bh * nt;
  const int b = bh / a.H, h = bh - b * a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sub = tid % LPR, d = 8 * sub;
  const bool din = d < a.D;  // columns past the head dim: zeros (the fp16 copy keeps D columns)
  const T* vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* qp = (const T*)a.q + b * a.sq[0] + h * a.sq[1];
  const T* op = (const T*)a.o + b * a.so[0] + h * a.so[1];
  const T* dop = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float* Lp = a.L + b * a.sl[0] + h * a.sl[1];
  i16x8 qv[NP];
  float qm = 0.f, vm = 0.f, am = 0.f, bm = 0.f;
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int row = 64 * t + RPP * u + tid / LPR;
    qv[u] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    float vs = 0.f, dsum = 0.f, dsq = 0.f;
    if (row < a.T && din) {
      // every input row is read once here: non-temporal loads (streamed, not
      // kept in L2)
      qv[u] = ld_nt16(qp + (int64_t)row * a.sq[2] + d);
      const VecT<T, 8> v8 = __builtin_bit_cast(VecT<T, 8>, ld_nt16(vp + (int64_t)row * a.sv[2] + d));
      const VecT<T, 8> o8 = __builtin_bit_cast(VecT<T, 8>, ld_nt16(op + (int64_t)row * a.so[2] + d));
      const VecT<T, 8> g8 = __builtin_bit_cast(VecT<T, 8>, ld_nt16(dop + (int64_t)row * a.sdo[2] + d));
      qm = fmaxf(qm, absmax8<T>(qv[u]));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vs = fmaf((float)v8.v[e], (float)v8.v[e], vs);
        dsum = fmaf((float)g8.v[e], (float)o8.v[e], dsum);
        dsq = fmaf((float)g8.v[e], (float)g8.v[e], dsq);
      }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
      vs += __shfl_xor(vs, o, 64);
      dsum += __shfl_xor(dsum, o, 64);
      dsq += __shfl_xor(dsq, o, 64);
    }
    vm = fmaxf(vm, sqrtf(vs));
    // the tile's stats: rows past T get zeros (the dK/dV kernel DMAs whole
    // 512-byte tiles, and a zero factor keeps its padding rows finite)
    float* st = ws.stats + ((int64_t)bh * nt + t) * 128 + (row & 63);
    if (row < a.T) {
      const float c4u = 1.f / (4.f * (Lp[(int64_t)row * a.sl[2]] + a.eps));
      if (sub == 0) {
        st[0] = c4u;
        st[64] = -c4u * dsum;
      }
      const float cw = fminf(4.1f, 1.125f * c4u);
      am = fmaxf(am, cw * sqrtf(dsq));
      bm = fmaxf(bm, cw * fabsf(dsum));
    } else if (sub == 0) {
      st[0] = 0.f;
      st[64] = 0.f;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    qm = fmaxf(qm, __shfl_xor(qm, o, 64));
    vm = fmaxf(vm, __shfl_xor(vm, o, 64));
    am = fmaxf(am, __shfl_xor(am, o, 64));
    bm = fmaxf(bm, __shfl_xor(bm, o, 64));
  }
  if (lane == 0) {
    red[0][w] = qm;
    red[1][w] = vm;
    red[2][w] = am;
    red[3][w] = bm;
  }
  __syncthreads();
  float m[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) m[i] = fmaxf(fmaxf(red[i][0], red[i][1]), fmaxf(red[i][2], red[i][3]));
  const int eq = tile_exp(m[0]);
  const float fq = ldexpf(1.f, eq);
  f16* qq = ws.q16 + (int64_t)bh * a.T * D;
  // non-temporal stores: the copy is read back only by the later kernels
  // (measured 0.3-0.9% faster over the backward than write-back stores)
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int row = 64 * t + RPP * u + tid / LPR;
    if (row < a.T) {
      __builtin_nontemporal_store(to_f16x8s<T>(qv[u], fq), reinterpret_cast<i16x8*>(qq + (int64_t)row * D + d));
    }
  }
  if (tid == 0) {
    ws.qexp[blockIdx.x] = eq;
    ws.vnrm[blockIdx.x] = m[1];
    ws.abnd[blockIdx.x] = m[2];
    ws.bbnd[blockIdx.x] = m[3];
  }
}

// dS exponents, one per 64-query tile t. kh = ds_exp(abnd_max vnrm_max +
// bbnd_max) is the exponent of the head's bound and e_t = ds_exp(abnd_t
// vnrm_max + bbnd_t) >= kh that of the tile's, so that every 2^e_t dS of the
// tile's rows lies below 2^14. A tile takes kq_t = kh + 8 floor((e_t - kh) / 8),
// capped at kh + kTileExpSpan: kh while its bound lies within 2^8 of the
// head's (its dS then reach fp16's subnormal range only 19 binades below their
// own bound), so that the dK accumulators, rescaled whenever the exponent
// changes from one query tile to the next, are rescaled only between tiles of
// very different magnitude; the cap bounds the factor of such a rescale. The
// per-row stats are multiplied by 2^kq_t in place (exact), so that
// dS = w (stats.x dP + stats.y) comes out scaled. Blocks of 256 rows of one
// head; each reduces the head's tile values itself (no atomics, no ordering
// between blocks) and records the exponents of its own tiles.
constexpr int kTileExpSpan = 40;  // a multiple of 8

template <int = 0>
__global__ __launch_bounds__(256) void attn_bwd_stscale_k(BwdWs ws, int T, int cpb) {
  __shared__ float red[3][4];
  const int nt = (T + 63) / 64;
  const int bh = (int)(blockIdx.x / (unsigned)cpb), ch = (int)blockIdx.x - bh * cpb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float vm = 0.f, am = 0.f, bm = 0.f;
  for (int i = tid; i < nt; i += 256) {
    const int64_t x = (int64_t)bh * nt + i;
    vm = fmaxf(vm, ws.vnrm[x]);
    am = fmaxf(am, ws.abnd[x]);
    bm = fmaxf(bm, ws.bbnd[x]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    vm = fmaxf(vm, __shfl_xor(vm, o, 64));
    am = fmaxf(am, __shfl_xor(am, o, 64));
    bm = fmaxf(bm, __shfl_xor(bm, o, 64));
  }
  if (lane == 0) {
    red[0][w] = vm;
    red[1][w] = am;
    red[2][w] = bm;
  }
  __syncthreads();
  vm = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  am = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  bm = fmaxf(fmaxf(red[2][0], red[2][1]), fmaxf(red[2][2], red[2][3]));
  const int kh = ds_exp(fmaf(am, vm, bm));
  const int r = 256 * ch + tid;
  if (r < T) {
    const int64_t t = (int64_t)bh * nt + (r >> 6);
    const int kq = kh + std::min((ds_exp(fmaf(ws.abnd[t], vm, ws.bbnd[t])) - kh) & ~7, kTileExpSpan);
    if ((r & 63) == 0) ws.ktile[t] = kq;
    const float f = ldexpf(1.f, kq);
    float* st = ws.stats + t * 128 + (r & 63);
    st[0] *= f;
    st[64] *= f;
  }
}

// ============================================================================
// dS^T tiles. The dK / dV kernel stores the fp16 dS it feeds its dK product
// (2^kq dS, zero where a key is masked or past its query) for every 64-key x
// 64-query tile (kt, qt) the backward touches, 8 KB each. Tiles are grouped by
// the dQ kernel's blocks of kQB query tiles so that each dQ block streams one
// contiguous run: a head's runs follow each other by query block qb, and
// within a run come, key tile by key tile (kt = 0 .. the block's last, causal;
// every kt otherwise), the block's kQB query tiles side by side (in causal
// mode the tiles with kt > qt inside a run are not written and not read).
// Long sequences whose tiles exceed the workspace's cap run in bands of key
// tiles [kb0, kb0 + nk) (kb0 and nk multiples of kQB, the last band shorter):
// a band keeps the same layout restricted to its key tiles, with runs for the
// query blocks that hold any of them (causal: qb >= kb0 / kQB). The whole head
// is the band kb0 = 0, nk = nt.
// Logically a tile is 64 key rows x 64 query columns; within each 32-query
// half the columns follow the dK kernel's MFMA operand order (column
// 8 g + 4 h + j holds query 16 h + 4 g + j). It is stored as eight 1 KB
// blocks, one per (32-key half kh2, 32-query half qh, 16-key group ks), at
// block (4 kh2 + 2 qh + ks): the 16-byte piece (key row 16 ks + i, columns
// 8 g .. 8 g + 7 of the query half) at position 16 g + i, i.e. exactly what
// lane (g, i) of the dK kernel's wave holds, so that each of its stores
// writes 1 KB contiguously (16 half-lines of 64 bytes took 4% longer over the
// backward). A 32-key half (one dQ stage) is the tile's first or second
// contiguous 4 KB, which the dQ kernel's DMA permutes back into row order.
// ============================================================================
constexpr int kQB = 8;  // 64-query tiles per dQ block

// first tile of query block qb's run in the band [kb0, kb0 + nk): causal runs
// hold min(nk, kQB (qb + 1) - kb0) key tiles (the last run: nk), the others nk
__host__ __device__ inline int64_t ds_run_base(int qb, bool causal, int kb0, int nk) {
  if (!causal) return (int64_t)qb * kQB * nk;
  const int64_t m = qb - kb0 / kQB, f = nk / kQB;
  const int64_t s = m <= f ? kQB * m * (m + 1) / 2 : kQB * f * (f + 1) / 2 + (m - f) * nk;
  return kQB * s;
}
__host__ __device__ inline int64_t ds_tiles_per_band(int nt, bool causal, int kb0, int nk) {
  const int nqb = (nt + kQB - 1) / kQB;
  return ds_run_base(nqb - 1, causal, kb0, nk) + (int64_t)kQB * nk;
}
__device__ __forceinline__ int64_t ds_tile(int kt, int qt, bool causal, int kb0, int nk) {
  return ds_run_base(qt / kQB, causal, kb0, nk) + (int64_t)(kt - kb0) * kQB + qt % kQB;
}
// query (0..31, within its half-tile) of column c of the half-tile
__device__ __forceinline__ int ds_col_query(int c) { return 16 * ((c >> 2) & 1) + 4 * (c >> 3) + (c & 3); }

// ============================================================================
// dQ from the stored dS: 512 queries (kQB 64-query tiles) per block, 8 waves,
// each owning one 64-query tile, one block per CU; per 32-key half of a key
// tile
//   dQ^T[d][q] += K16^T[d][key] dS^T[key][q]   A = K16^T (LDS transposed)
//                                              B = dS^T  (LDS transposed)
// A plain GEMM, bound by streaming the stored dS once. Each wave stages its
// own dS rows (from the block's contiguous run, non-temporal LDS-DMA) and the
// block shares the K rows, 32 keys per stage, four stages deep (two in flight
// while one is worked and one is converted); a stage issues the same number
// of DMA instructions per wave whatever it holds (rows a wave does not need
// come through an empty resource: zeros, no memory access), so that one vmcnt
// value waits for the oldest stage. The K rows come in the input dtype and
// are converted in LDS, one stage ahead, to the fp16 copy K16 = K 2^ek that
// the dK/dV kernel formed for the same 32 keys (ek: its exponent, read from
// kexp; the conversion is the same function, so K16 is bit-identical): the
// backward keeps no fp16 copy of K in HBM, and this kernel's spare VALU does
// the conversion. Each K16 fragment read from LDS feeds four MFMAs. Blocks
// take the forward's order (heads pinned to XCDs, longest blocks first across
// the XCD's heads). dS carries its query tile's 2^kq and K16 its 32 keys'
// 2^ek: the accumulators are rescaled when ek changes and the epilogue
// multiplies by scale 2^-(kq + ek) (exact). Blocks cover the heads
// bh0 .. bh0 + G - 1 (the dS tiles in the workspace) and the key tiles of the
// band [kb0, kb0 + nk): a wave whose queries see keys before the band starts
// from its fp32 partial sums in dqacc, and one whose queries see keys after it
// leaves its partial sums there (divided by 2^ek, exact) instead of writing
// dQ; the bands run in order, so the sums are added in a fixed order.
// ============================================================================
constexpr int kDqW = kQB;           // waves per dQ block
constexpr int kDqS = 4;             // stages (32 keys each)
// queries per dQ wave: a 64-query tile, or at D = 256 (whose accumulators for
// 64 queries would take all 256 VGPRs) a 32-query half of one; a block covers
// kDqW waves' queries, i.e. a whole dS run (kQB tiles) or half of one
template <int D> constexpr int dq_qw() { return D == 256 ? 32 : 64; }
template <int D> constexpr int dq_block_queries() { return kDqW * dq_qw<D>(); }

template <int D> struct DqSmem {
  short k[kDqS][32 * D];                   // K rows (converted in place to K16)
  short s[kDqS][kDqW][32 * dq_qw<D>()];    // each wave's dS^T rows
};

template <typename T, int D, int MODE, int DE = D>
__global__ __launch_bounds__(64 * kDqW, 1) void attn_bwd_dq_k(AttnArgs a, const int* __restrict__ kexp,
                                                              const int* __restrict__ ktile,
                                                              const f16* __restrict__ dst, int bh0, int G,
                                                              int kb0, int nk, float* __restrict__ dqacc) {
  typedef Mfma<T> M;
  constexpr int DS = DE / 16;
  constexpr int QW = dq_qw<D>(), QC = QW / 16;  // queries per wave, 16-query column groups
  constexpr int BQ = dq_block_queries<D>();      // queries per block
  constexpr int WPT = 64 / QW;                   // waves per 64-query tile
  constexpr bool kCausal = (MODE & kModeCausal) != 0;
  // K16 rows: 1 KB DMA segments over the first KW waves (all 8 at D = 128,
  // 4 at D = 64); dS rows: each wave its own
  constexpr int KW = std::min(kDqW, 32 * D / 512);
  typedef TileDma<D, KW, 32> KDma;
  typedef TileDma<QW, 1, 32> SDma;
  __shared__ DqSmem<D> sm;

  const int T_ = a.T, H = a.H;
  const int n_qb = (T_ + BQ - 1) / BQ;
  int bl, rank;
  block_order((int)blockIdx.x, G, bl, rank);
  const int bh = bh0 + bl;
  const int qb = n_qb - 1 - rank;
  const int q0 = qb * BQ;
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int g = lane >> 4, li = lane & 15;
  const int nt = (T_ + 63) / 64;
  const int qtw = (q0 >> 6) + w / WPT;      // this wave's 64-query tile
  const int qh = WPT == 1 ? 0 : w % WPT;    // and its 32-query half (QW = 32)
  const int tir = qtw % kQB;                // the tile's place in its dS run
  const bool wact = qtw < nt;
  const T* kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const uint32_t sk2 = (uint32_t)a.sk[2];
  const int DR = a.D;  // the head dim (<= D; columns DR .. D - 1 read as zeros, not stored)
  const uint32_t kbytes = row_bytes(T_, sk2, DR);
  const f16* run = dst + ((int64_t)bl * ds_tiles_per_band(nt, kCausal, kb0, nk) +
                           ds_run_base(q0 / (kQB * 64), kCausal, kb0, nk)) * 4096;
  const int ng = (T_ + 31) / 32;  // 32-key groups (exponents)
  const int* kexp_h = kexp + (int64_t)bh * ng;
  const int kt_all = kCausal ? std::min((q0 >> 6) + BQ / 64, nt) : nt;  // the block's key tiles: 0 .. kt_all - 1
  const int kt_end = std::min(kb0 + nk, kt_all);
  const int n_st = 2 * (kt_end - kb0);      // stages: 32-key halves of the band's key tiles
  float* const part = dqacc + (((int64_t)bl * nt + qtw) * 64 + qh * QW) * D;  // this wave's partial sums
  const bool kw_ = w < KW;
  const int ndma = (kw_ ? KDma::SEGS : 0) + SDma::SEGS;  // this wave's DMA per stage

  f32x4 acc[DS][QC];  // [d subtile][16-query column group]
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int qc = 0; qc < QC; ++qc) acc[ds][qc] = f32x4{0.f, 0.f, 0.f, 0.f};

  KDma dk;
  SDma dd;  // the wave's own dS rows
  dk.init(kw_ ? w : 0, lane, sk2, DR);
  // LDS slot (row, p) of the swizzled [32][QW] stage tile takes data chunk
  // c = p ^ swz(row) of key row `row`, which the stored layout keeps in 1 KB
  // block 2 (c / 4) + row / 16 at position 16 (c % 4) + row % 16 (QW = 32:
  // the 32-query half's two blocks, qh's 2 KB of the stage)
#pragma unroll
  for (int u = 0; u < SDma::SEGS; ++u) {
    const int row = u * SDma::RPS + lane / SDma::CPR;
    const int c = (lane % SDma::CPR) ^ swz<QW>(row);
    dd.off[u] = (uint32_t)((((c >> 2) * 2 + (row >> 4)) * 64 + 16 * (c & 3) + (row & 15)) * 16);
  }
  auto tile_in = [&](int kt) __attribute__((always_inline)) { return wact && (!kCausal || kt <= qtw); };
  // stage st: rows 32 (st & 1) .. of key tile kb0 + (st >> 1)
  auto issue = [&](int buf, int st) __attribute__((always_inline)) {
    const int kl = st >> 1;
    if (kw_) dk.issue(sm.k[buf], kp, kbytes, 32 * (2 * kb0 + st), sk2, w);
    const bool have = tile_in(kb0 + kl);
    dd.template issue<true>(sm.s[buf][w], run + (have ? ((int64_t)kl * kQB + tir) * 4096 + qh * 1024 : 0),
                            have ? 8192u - 2048u * qh : 0u, 32 * (st & 1), 64, 0);
  };
  // stage st has landed when at most the stages issued after it (up to `ahead`
  // of them) are in flight (loads complete in order); the count is an immediate
  constexpr int kA = KDma::SEGS + SDma::SEGS, kB = SDma::SEGS;
  auto wait_for = [&](int st, int ahead) __attribute__((always_inline)) {
    const int after = std::min(n_st - 1 - st, ahead) * ndma;
    if (after == 2 * kA) __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * kA));
    else if (after == kA) __builtin_amdgcn_s_waitcnt(0x0F70 | kA);
    else if (after == 2 * kB) __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * kB));
    else if (after == kB) __builtin_amdgcn_s_waitcnt(0x0F70 | kB);
    else dma_wait();
  };
  // exponent of stage st's 32 keys (a stage past the last key group holds only
  // zero rows: any exponent serves)
  auto stage_exp = [&](int st) __attribute__((always_inline)) { return kexp_h[std::min(2 * kb0 + st, ng - 1)]; };
  // stage st's K rows to K16 in place: one 16-byte chunk per thread
  auto convert = [&](short* kt_, int st) __attribute__((always_inline)) {
    const float f = ldexpf(1.f, stage_exp(st));
#pragma unroll
    for (int c = tid; c < 32 * D / 8; c += 64 * kDqW) {
      i16x8* p = reinterpret_cast<i16x8*>(kt_ + 8 * c);
      *p = to_f16x8s<T>(*p, f);
    }
  };
  int ek = 0;
  if (kb0 > 0 && wact) {
    // the partial sums of the earlier bands (lane order, as stored below),
    // complete before the first DMA is issued: with these loads pending at
    // the loop, the compiler's own waits there would also wait for the DMA
    // issued ahead (measured: the kernel 40% slower)
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
#pragma unroll
      for (int qc = 0; qc < QC; ++qc) acc[ds][qc] = *reinterpret_cast<const f32x4*>(part + ((ds * QC + qc) * 64 + lane) * 4);
    dma_wait();
  }
  for (int st = 0; st < kDqS - 1; ++st)
    if (st < n_st) issue(st, st);
  wait_for(std::min(1, n_st - 1), 1);
  __syncthreads();
  convert(sm.k[0], 0);
  if (n_st > 1) convert(sm.k[1], 1);
  __syncthreads();
  // unrolled by four: static buffers
  auto step = [&](int st, auto buf_tag) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_tag)::value;
    if (st + kDqS - 1 < n_st) issue((buf + kDqS - 1) % kDqS, st + kDqS - 1);
    const int kt = kb0 + (st >> 1);
    const int est = stage_exp(st);
    if (est != ek) {
      const float f = ldexpf(1.f, est - ek);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
#pragma unroll
        for (int qc = 0; qc < QC; ++qc) acc[ds][qc] *= f;
      ek = est;
    }
    if (tile_in(kt)) {
      const short* sd = sm.s[buf][w];
      i16x8 bq[QC];
#pragma unroll
      for (int qc = 0; qc < QC; ++qc) bq[qc] = frag_tr<QW>(sd, 0, 16 * qc, g, li);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const i16x8 at = frag_tr<D>(sm.k[buf], 0, 16 * ds, g, li);
#pragma unroll
        for (int qc = 0; qc < QC; ++qc) acc[ds][qc] = mma_f16(at, bq[qc], acc[ds][qc]);
      }
    }
    // the stage after the next has landed (the next is converted), and every
    // wave is done with this stage's buffers
    if (st + 2 < n_st) wait_for(st + 2, 1);
    __syncthreads();
    // its K rows to K16 (read by step st + 2, after the next barrier)
    if (st + 2 < n_st) convert(sm.k[(buf + 2) % kDqS], st + 2);
  };
  for (int st = 0; st < n_st; st += 4) {
    step(st, std::integral_constant<int, 0>{});
    step(st + 1, std::integral_constant<int, 1>{});
    if (st + 2 < n_st) {
      step(st + 2, std::integral_constant<int, 2>{});
      step(st + 3, std::integral_constant<int, 3>{});
    }
  }

  if (kt_end < kt_all) {
    // keys after the band remain: keep the partial sums, with ek taken out
    if (wact) {
      const float f = ldexpf(1.f, -ek);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
#pragma unroll
        for (int qc = 0; qc < QC; ++qc)
          *reinterpret_cast<f32x4*>(part + ((ds * QC + qc) * 64 + lane) * 4) = acc[ds][qc] * f;
    }
    return;
  }
  T* __restrict__ dqp = (T*)a.dq + b * a.sdq[0] + h * a.sdq[1];
  const float osc = ldexpf(a.scale, -((wact ? ktile[(int64_t)bh * nt + qtw] : 0) + ek));
  // the wave's QW query rows through its own QW x D staging tile in the
  // (now idle) stage buffers
  static_assert(sizeof(sm) >= kDqW * QW * D * 2, "staging tiles fit the stage buffers");
  short* const et = reinterpret_cast<short*>(&sm) + w * QW * D;
#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    // column 16 qc + li of the wave's queries: 32-query half (qc >> 1), column
    // 16 (qc & 1) + li in it
    const int r = 32 * (qc >> 1) + ds_col_query(16 * (qc & 1) + li);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const f32x4 o = acc[ds][qc];
      epi_put(et, eoff<D>(r, 16 * ds + 4 * g), M::pack2(o[0] * osc, o[1] * osc), M::pack2(o[2] * osc, o[3] * osc));
    }
  }
  __syncthreads();  // orders the tile's writes before its reads
  epi_rows_out<T, D, QW>(et, lane, dqp, a.sdq[2], 64 * qtw + QW * qh, T_, DR);
}

// ============================================================================
// dK, dV: 4 KR keys per block, 8 waves in two roles. Waves w and w + 4 share the
// KR keys kw = k0 + KR (w % 4) and one SIMD (KR = 32 at D = 128, see
// dkv_keys); each role holds one B-operand set and one accumulator set
// (~200 VGPRs, two waves per SIMD):
//   P role (w < 4)   S  = Q16 K16^T (+bias)  A = Q16 (LDS rows)         B = K16^T (VGPRs)
//                    dV^T += dO^T P          A = dO^T (LDS transposed)  B = P (from S)
//   D role (w >= 4)  dP = dO V^T             A = dO  (LDS rows)         B = V^T   (VGPRs)
//                    dK^T += Q16^T dS        A = Q16^T (LDS transposed) B = dS
// The P role also forms w = (t r)^2 t of every score and passes it to the D role
// through LDS, lane to lane (both roles hold the scores of a 16-query half in
// the same MFMA C layout), so dS = w (4 cinv dP - 4 cinv Delta) costs the D role
// one FMA and one multiply. (Passing t instead and forming w in the D role,
// from r = min(t, 2 - t), splits the VALU work evenly between the waves but
// costs two more operations per score and measured 1-2% slower: the SIMD's
// instruction issue, not either wave's chain, bounds this kernel.)
// 64-query Q16 / dO tiles and their stats stream
// through LDS; a tile is worked in two 32-query chunks with one barrier each:
//   phase 1: P role S, P, w of chunk c                    | barrier
//   phase 2: P role dV(c); D role dP(c + 1), dS(c), dK(c)
// The D role computes dP one chunk ahead (KR = 32) so that the reads of w
// issued after the barrier overlap with MFMAs.
// ============================================================================
template <int D, int KS>
struct DkvSmem {
  short q[2][kBN * D];         // Q16 tiles
  short o[2][kBN * D];         // dO tiles
  f32x4 x[2][kNW][2 * KS][64];  // w: [chunk parity][key group][16-query half x ks][lane]
  float st[2][2 * kBN];        // the tile's stats: 4 cinv of its queries, then -4 cinv Delta
  float km[kNW];               // KS = 1: the key groups' max |k| (pairs share an exponent)
};

// KR: keys per wave pair. 32 at D = 32 and 128; 64 at D = 64 (twice the
// MFMAs per LDS read of the streamed Q16 / dO tiles, in the registers D = 128
// takes for 32 keys: backward 9-10% faster than 32 keys; at D = 32, whose
// time is the per-score VALU work, 64 keys measured 10-13% slower); 16 at
// D = 256 (whose B fragments and accumulators of 32 keys would exceed the
// register budget), the two pairs of a 32-key group then sharing one K16
// exponent. K16 exponents are per 32 keys at every KR.
template <int D> constexpr int dkv_keys() { return D == 256 ? 16 : D == 64 ? 64 : kRows; }
template <typename T, int D, int MODE, int KR = kRows, int DE = D>
__global__ __launch_bounds__(512, 1) void attn_bwd_dkv_k(AttnArgs a, const float* __restrict__ stats,
                                                         const f16* __restrict__ q16,
                                                         const int* __restrict__ qexp,
                                                         const int* __restrict__ ktile,
                                                         int* __restrict__ kexp,
                                                         f16* __restrict__ dst, int bh0, int G, int kb0,
                                                         int nk) {
  typedef Mfma<T> M;
  constexpr int KK = DE / 32;
  constexpr int DS = DE / 16;
  constexpr bool kCausal = (MODE & kModeCausal) != 0;
  constexpr bool kKM = (MODE & kModeKeyMask) != 0;
  constexpr int KS = KR / 16;     // 16-key groups per wave
  constexpr int NE = (KS + 1) / 2;  // K16 exponents per wave (one per 32 keys; 16-key group ks takes ks / 2)
  constexpr int BK = kNW * KR;    // keys per block
  __shared__ DkvSmem<D, KS> sm;

  const int T_ = a.T, H = a.H;
  int bl, rank;
  block_order((int)blockIdx.x, G, bl, rank);  // rank 0: the first keys (most queries)
  const int bh = bh0 + bl;
  const int k0 = kb0 * 64 + rank * BK;  // blocks cover the band's keys
  const int b = bh / H, h = bh - b * H;
  // the key group (and the tile conditions derived from it) as scalars; the
  // role test stays a per-lane value: as a scalar branch the two roles' code
  // no longer fits 256 VGPRs (spills)
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int grp = w % kNW;
  const bool prole = (tid >> 6) < kNW;
  const int g = lane >> 4, li = lane & 15;
  const int kw = k0 + KR * grp;

  const f16* qp = q16 + (int64_t)bh * T_ * D;
  const T* kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1];
  const T* vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1];
  const T* dop = (const T*)a.dout + b * a.sdo[0] + h * a.sdo[1];
  const float* stp = stats + (int64_t)bh * ((T_ + 63) / 64) * 128;
  const uint32_t sk2 = (uint32_t)a.sk[2], sv2 = (uint32_t)a.sv[2], sdo2 = (uint32_t)a.sdo[2];
  const int DR = a.D;  // the head dim (<= D; columns DR .. D - 1 read as zeros, not stored)
  const uint32_t qbytes = row_bytes(T_, D, D), obytes = row_bytes(T_, sdo2, DR);
  const uint32_t stbytes = (uint32_t)((T_ + 63) / 64) * 512u;
  const float slope = a.slopes[h];
  const float scale = a.scale;
  // the stats carry their tile's dS exponent (stats.x = 2^kq 4 cinv); P takes
  // 4 cinv / 16 = cinv / 4, i.e. stats.x p4 with p4 = 2^-kq / 4 (set per tile)
  float p4 = 0.25f;
  const int nt = (T_ + 63) / 64;
  const int* qexp_h = qexp + (int64_t)bh * nt;
  const int* ktile_h = ktile + (int64_t)bh * nt;
  // D role: where this wave's dS^T goes (lane (g, li) of half-tile row
  // 16 ks + li, columns 8 g .. 8 g + 7); tiles past the head's last are not kept
  const int ktg = kw >> 6;
  const bool dst_ok = ktg < nt;
  f16* const dsh = dst + (int64_t)bl * ds_tiles_per_band(nt, kCausal, kb0, nk) * 4096;
  // block 4 kh2 + 2 qh + kg of the tile (kh2: the 32-key half, kg: the
  // 16-key group within it); dso[ks]: the offset of 16-key group ks's block
  // (without the 32-query half qh) plus the lane's 16 bytes
  uint32_t dso[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int ko = (kw & 63) + 16 * ks;
    dso[ks] = (uint32_t)((ko >> 5) * 2048 + ((ko >> 4) & 1) * 512 + lane * 8);
  }
  f16* dtile = dsh;  // the current query tile's dS^T tile

  // B operands: K16^T (P role) or V^T (D role) fragments; lane (g, li) holds row
  // kw + 16 ks + li, columns 32 kk + 8 g .. +7
  // (P role: scaled by 2^ekw[ks / 2], the exponent tile_exp gives their 32 keys)
  i16x8 bfr[KS][KK];
  int ekw[NE];
  {
    const __amdgpu_buffer_rsrc_t rk = rsrc(kp, row_bytes(T_, sk2, DR));
    const __amdgpu_buffer_rsrc_t rv = rsrc(vp, row_bytes(T_, sv2, DR));
    float km[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      km[e] = 0.f;
      ekw[e] = 0;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint32_t key = (uint32_t)(kw + 16 * ks + li);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int col = 32 * kk + 8 * g;
        if (prole) {
          bfr[ks][kk] = load16(rk, col_off((key * sk2 + col) * 2, col, DR));
          km[ks / 2] = fmaxf(km[ks / 2], absmax8<T>(bfr[ks][kk]));
        } else {
          bfr[ks][kk] = load16(rv, col_off((key * sv2 + col) * 2, col, DR));
        }
      }
    }
    if (prole) {
#pragma unroll
      for (int e = 0; e < NE; ++e)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) km[e] = fmaxf(km[e], __shfl_xor(km[e], o, 64));
    }
    if constexpr (KS == 1) {
      // the 32-key group's two 16-key halves (waves grp and grp ^ 1) share one
      // exponent: the max of both
      if (prole && lane == 0) sm.km[grp] = km[0];
      __syncthreads();
      if (prole) km[0] = fmaxf(km[0], sm.km[grp ^ 1]);
    }
    if (prole) {
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        ekw[e] = tile_exp(km[e]);
        // the dQ kernel converts these 32 keys with the same exponent
        if (lane == 0 && kw + 32 * e < T_ && (KS >= 2 || (grp & 1) == 0))
          kexp[(int64_t)bh * ((T_ + 31) / 32) + (kw >> 5) + e] = ekw[e];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const float fk = ldexpf(1.f, ekw[ks / 2]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) bfr[ks][kk] = to_f16x8s<T>(bfr[ks][kk], fk);
      }
    }
  }
  // S layout: lane (g, li) element j holds q = qh + 4 g + j, key = kw + 16 ks + li
  f32x4 cb;
#pragma unroll
  for (int j = 0; j < 4; ++j) cb[j] = (slope / scale) * (float)(li - 4 * g - j);
  // bias in use (negated for query chunks wholly below this wave's keys in
  // non-causal mode). S comes out of the MFMA scaled by 2^(eq + ekw) (eq: the
  // Q16 tile's exponent): cbx carries that factor and sc = scale 2^-(eq + ekw)
  // removes it (one of each per K16 exponent); the dK accumulators hold
  // 2^(eq + kq) times the sum (kq: the query tile's dS exponent), rescaled
  // when a tile brings other exponents.
  int eq = 0, kq = 0;
  float sfac[NE], sc[NE];  // 2^(eq + ekw), scale 2^-(eq + ekw)
  f32x4 cbx[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    sfac[e] = ldexpf(1.f, ekw[e]);
    cbx[e] = cb * sfac[e];
    sc[e] = ldexpf(scale, -ekw[e]);
  }
  float slx = slope;
  // Padding mask: a dropped key's P and dS column is zero, so its dK / dV
  // rows are zero and the other keys' rows do not depend on it. The kernel
  // computes every key and stores zeros for dropped ones; a wave pair whose
  // KR keys are all dropped skips the work.
  bool kval[KS];
  bool gany = true;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kval[ks] = true;
  if constexpr (kKM) {
    const uint8_t* kmb = a.km + (int64_t)b * a.skm;
    bool any = false;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int key = kw + 16 * ks + li;
      kval[ks] = key < T_ && kmb[key] != 0;
      any = any || kval[ks];
    }
    gany = __builtin_amdgcn_ballot_w64(any) != 0ull;
  }

  f32x4 acc[DS][KS];  // dV^T (P role) or dK^T (D role)
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) acc[ds][ks] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the P role's waves stage the tiles: the D role's waves then have no loads
  // in flight inside the loop and never wait for their dS stores
  TileDma<D, kNW> dq_, do_;
  dq_.init(w, lane, D);
  do_.init(w, lane, sdo2, DR);
  // stats of a 64-query tile: 512 bytes, lanes 0..31 of wave 0
  const uint32_t st_off = (uint32_t)lane * 16u;
  auto issue = [&](int buf, int qrow0) __attribute__((always_inline)) {
    if (prole) {
      dq_.issue(sm.q[buf], qp, qbytes, qrow0, D, w);
      do_.issue(sm.o[buf], dop, obytes, qrow0, sdo2, w);
    }
    if (w == 0 && lane < 32) {
      const uint32_t skip = (uint32_t)qrow0 * 8u;  // qrow0 is a multiple of 64: 512 bytes per tile
      dma16(rsrc_words((const char*)stp + skip, stbytes > skip ? stbytes - skip : 0u), lds_addr(sm.st[buf]),
            st_off);
    }
  };

  // S (P role) or dP (D role) of the 16 queries at tile rows hr .. hr + 15
  auto m1 = [&](auto role, int hr, f32x4 (&s_)[KS], const short* as_) __attribute__((always_inline)) {
    constexpr bool P = decltype(role)::value;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s_[ks] = P ? cbx[ks / 2] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const i16x8 fa = lds16(as_ + soff<D>(hr + li, 32 * kk + 8 * g));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (P) s_[ks] = mma_f16(fa, bfr[ks][kk], s_[ks]);
        else s_[ks] = M::mma(fa, bfr[ks][kk], s_[ks]);
      }
    }
  };
  // P role: P (input dtype) of a 16-query half, and w into the exchange buffer.
  // DIAG: a chunk that straddles the diagonal (causal: keys past the query get
  // P = w = 0; non-causal: their bias becomes -slope (key - q)).
  auto vp_ = [&](auto diag_tag, int qh, int hr, const f32x4 (&s_)[KS], const float* st_, f32x4 (*xw)[64],
                 int xg, uint32_t (&pp)[KS][2]) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const f32x4 c4v = *reinterpret_cast<const f32x4*>(st_ + hr + 4 * g);  // 4 cinv of queries hr + 4 g + j
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const float tterm = slx * (float)(kw + 16 * ks - qh);
      float pv[4];
      f32x4 wv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float s = fmaf(s_[ks][j], sc[ks / 2], tterm);
        if constexpr (DIAG && !kCausal) {
          const int dkq = (kw + 16 * ks + li) - (qh + 4 * g + j);
          if (dkq > 0) s = fmaf(-2.f * slope, (float)dkq, s);
        }
        const float r = __builtin_amdgcn_rcpf(fabsf(s) + 1.f);
        const float t = fmaf(s, r, 1.f);
        const float t2 = t * t;
        const float u = t * r;
        pv[j] = (t2 * t2) * (p4 * c4v[j]);
        wv[j] = u * u * t;
        if (DIAG && kCausal && kw + 16 * ks + li > qh + 4 * g + j) {
          pv[j] = 0.f;
          wv[j] = 0.f;
        }
      }
      xw[xg + ks][lane] = wv;
      pp[ks][0] = M::pack2(pv[0], pv[1]);
      pp[ks][1] = M::pack2(pv[2], pv[3]);
    }
  };
  // acc^T += A^T B over the 32 queries at tile rows r0 .. r0 + 31, A = dO (P role)
  // or Q16 (D role) read transposed, B = P or dS
  auto m2 = [&](auto role, int r0, const uint32_t (&pa)[KS][2], const uint32_t (&pb)[KS][2],
                const short* as_) __attribute__((always_inline)) {
    constexpr bool P = decltype(role)::value;
    i16x8 bf2[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) bf2[ks] = pack_frag(pa[ks][0], pa[ks][1], pb[ks][0], pb[ks][1]);
    i16x8 at[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) at[ds] = frag_tr<D>(as_, r0, 16 * ds, g, li);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (P) acc[ds][ks] = M::mma(at[ds], bf2[ks], acc[ds][ks]);
        else acc[ds][ks] = mma_f16(at[ds], bf2[ks], acc[ds][ks]);
      }
    }
    // the transposed reads run one pair of d-subtiles ahead of the MFMAs that
    // take them (0x100: LDS reads, 0x008: MFMA)
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int st = 0; st < DS / 2 - 1; ++st) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * KS, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * KS, 0);
  };

  // chunk c: queries qbase + 32 c .. +31, tile (c / 2) in buffer (c / 2) & 1,
  // rows 32 (c & 1); causal: queries from k0 on, non-causal: every query
  const int qbase = kCausal ? k0 : 0;
  const int n_it = qbase < T_ ? (T_ - qbase + kBN - 1) / kBN : 0;
  const int n_ch = 2 * n_it;
  auto needc = [&](int c) __attribute__((always_inline)) {
    return c < n_ch && gany && (!kCausal || qbase + 32 * c + 31 >= kw);
  };
  // no key of the wave lies past a query of the chunk (non-causal: or every key does)
  auto fullc = [&](int c) __attribute__((always_inline)) {
    return qbase + 32 * c >= kw + KR - 1 || (!kCausal && kw > qbase + 32 * c + 31);
  };
  if (n_it > 0) issue(0, qbase);
  if (prole) dma_wait();
  __syncthreads();
  // D role: dP of the current and the next chunk (KS = 2). At KS = 4 the
  // registers of the next chunk's dP do not fit beside the rest, and at KS = 1
  // (D = 256) they cost spills in the non-causal modes: dP is then computed in
  // its own step, after the barrier (its MFMAs cover the reads of w; D = 256
  // measured 0-3% faster causal and 8% non-causal, bit-identical)
  constexpr bool kAhead = KS == 2;
  f32x4 dpA[2][KS], dpB[2][KS];
  if (kAhead && !prole && needc(0)) {
    m1(std::false_type{}, 0, dpA[0], sm.o[0]);
    m1(std::false_type{}, 16, dpA[1], sm.o[0]);
  }
  // chunk c of the loop, with CM = c % 4 known at compile time (the loop is
  // unrolled by four), so that the tile buffer, the rows within it and the
  // exchange buffer -- and with them every LDS address -- are a per-lane
  // register plus an immediate
  auto step = [&](int c, auto cm_tag, f32x4 (&pcur)[2][KS], f32x4 (&pnext)[2][KS]) __attribute__((always_inline)) {
    constexpr int CM = decltype(cm_tag)::value;
    constexpr int buf = CM >> 1, r0 = 32 * (CM & 1);
    const int it = c >> 1;
    const int qc = qbase + 32 * c;
    const bool need = needc(c), full = need && fullc(c);
    f32x4 (*xw)[64] = sm.x[CM & 1][grp];
    uint32_t pa[KS][2], pb[KS][2];
    if constexpr ((CM & 1) == 0) {
      // a new query tile: its Q16 and dS exponents (both roles track them)
      const int eqt = qexp_h[(qbase >> 6) + it], kqt = ktile_h[(qbase >> 6) + it];
      if (eqt != eq) {
        const float f = ldexpf(1.f, eqt - eq);
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          sfac[e] *= f;
          sc[e] = ldexpf(sc[e], eq - eqt);
          if constexpr (kCausal) cbx[e] *= f;
        }
      }
      p4 = ldexpf(0.25f, -kqt);
      // D role: this query tile's dS^T tile (both of its chunks)
      dtile = dsh + ds_tile(ktg, (qbase >> 6) + it, kCausal, kb0, nk) * 4096;
      if (!prole && eqt + kqt != eq + kq) {
        const float f = ldexpf(1.f, (eqt + kqt) - (eq + kq));
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) acc[ds][ks] *= f;
      }
      eq = eqt;
      kq = kqt;
    }
    if constexpr (!kCausal) {
      const bool above = kw > qc + 31;
#pragma unroll
      for (int e = 0; e < NE; ++e) cbx[e] = (above ? -cb : cb) * sfac[e];
      slx = above ? -slope : slope;
    }
    if (prole && need) {
      f32x4 sA[KS], sB[KS];
      m1(std::true_type{}, r0, sA, sm.q[buf]);
      m1(std::true_type{}, r0 + 16, sB, sm.q[buf]);
      if (full) {
        vp_(std::false_type{}, qc, r0, sA, sm.st[buf], xw, 0, pa);
        vp_(std::false_type{}, qc + 16, r0 + 16, sB, sm.st[buf], xw, KS, pb);
      } else {
        vp_(std::true_type{}, qc, r0, sA, sm.st[buf], xw, 0, pa);
        vp_(std::true_type{}, qc + 16, r0 + 16, sB, sm.st[buf], xw, KS, pb);
      }
    }
    if constexpr ((CM & 1) == 0) {
      // every wave has left the previous tile: its buffer takes the next one
      __syncthreads();
      if (it + 1 < n_it) issue(buf ^ 1, qbase + (it + 1) * kBN);
    } else {
      // the next tile has landed (each P-role wave waits for its own DMA)
      if (prole) dma_wait();
      __syncthreads();
    }
    if (prole) {
      if (need) m2(std::true_type{}, r0, pa, pb, sm.o[buf]);
    } else {
      // w of this chunk (read whether or not the chunk is needed: the buffer
      // always exists, and a conditional read leaves the compiler zeroing the
      // registers on the other path every chunk)
      // (KS = 4: each half's w just before its use)
      f32x4 wv[2 * KS];
      if constexpr (kAhead) {
#pragma unroll
        for (int u = 0; u < 2 * KS; ++u) wv[u] = xw[u][lane];
      }
      if constexpr (kAhead) {
        if (needc(c + 1)) {
          constexpr int r1 = 32 * ((CM + 1) & 1);
          const short* os1 = sm.o[((CM + 1) >> 1) & 1];
          m1(std::false_type{}, r1, pnext[0], os1);
          m1(std::false_type{}, r1 + 16, pnext[1], os1);
        }
      } else if (need) {
        m1(std::false_type{}, r0, pcur[0], sm.o[buf]);
        m1(std::false_type{}, r0 + 16, pcur[1], sm.o[buf]);
      }
      if (need) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const f32x4 c4v = *reinterpret_cast<const f32x4*>(sm.st[buf] + r0 + 16 * hh + 4 * g);
          const f32x4 ndv = *reinterpret_cast<const f32x4*>(sm.st[buf] + kBN + r0 + 16 * hh + 4 * g);
          uint32_t (&dp)[KS][2] = hh ? pb : pa;
          if constexpr (!kAhead) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) wv[KS * hh + ks] = xw[KS * hh + ks][lane];
          }
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            float dv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              // w = t^3 r^2 from t alone: r = 1 / (|s| + 1) equals t for s < 0
              // and 2 - t for s >= 0, i.e. min(t, 2 - t) (exact given t)
              dv[j] = wv[KS * hh + ks][j] * fmaf(pcur[hh][ks][j], c4v[j], ndv[j]);
            }
            dp[ks][0] = pack2_f16(dv[0], dv[1]);
            dp[ks][1] = pack2_f16(dv[2], dv[3]);
          }
        }
        if constexpr (kKM) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            if (!kval[ks]) pa[ks][0] = pa[ks][1] = pb[ks][0] = pb[ks][1] = 0u;
        }
        // dS^T for the dQ kernel: 16 bytes per lane and ks (streaming stores:
        // the dQ kernel reads them back only after this kernel)
        if (dst_ok) {
          f16* const tb = dtile + (r0 >> 5) * 1024;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            __builtin_nontemporal_store(pack_frag(pa[ks][0], pa[ks][1], pb[ks][0], pb[ks][1]),
                                        reinterpret_cast<i16x8*>(tb + dso[ks]));
        }
        m2(std::false_type{}, r0, pa, pb, sm.q[buf]);
      } else if (dst_ok && c < n_ch && (!kCausal || (c >> 1) >= ((KR * grp) >> 6))) {
        // a skipped chunk inside a kept tile: its dS is zero
        f16* const tb = dtile + (r0 >> 5) * 1024;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          __builtin_nontemporal_store(i16x8{0, 0, 0, 0, 0, 0, 0, 0},
                                      reinterpret_cast<i16x8*>(tb + dso[ks]));
      }
    }
  };
  // unrolled by four (two tiles): static buffers, and the D role's dP
  // registers alternate; n_ch is even
  for (int c = 0; c < n_ch; c += 4) {
    step(c, std::integral_constant<int, 0>{}, dpA, dpB);
    step(c + 1, std::integral_constant<int, 1>{}, dpB, dpA);
    if (c + 2 < n_ch) {
      step(c + 2, std::integral_constant<int, 2>{}, dpA, dpB);
      step(c + 3, std::integral_constant<int, 3>{}, dpB, dpA);
    }
  }

  T* __restrict__ outp = prole ? (T*)a.dv + b * a.sdv[0] + h * a.sdv[1] : (T*)a.dk + b * a.sdk[0] + h * a.sdk[1];
  const int64_t ostr = prole ? a.sdv[2] : a.sdk[2];
  const float osc = prole ? 1.f : ldexpf(scale, -(kq + eq));  // dK: dS's 2^kq and Q16's 2^eq undone (exact)
  // the wave's KR rows (keys) through its own KR x D staging tile in the now
  // idle tile and exchange buffers (8 waves x KR x D x 2 bytes within the
  // Q16, dO and w buffers)
  typedef DkvSmem<D, KS> Smem;
  static_assert(sizeof(sm.q) + sizeof(sm.o) + sizeof(sm.x) >= 8 * KR * D * 2 && offsetof(Smem, q) == 0 &&
                    offsetof(Smem, o) == sizeof(sm.q) && offsetof(Smem, x) == sizeof(sm.q) + sizeof(sm.o),
                "staging tiles fit the tile and exchange buffers");
  short* const et = reinterpret_cast<short*>(&sm) + w * KR * D;
  __syncthreads();  // every wave is done with the tile buffers
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      f32x4 v = acc[ds][ks];
      if (kKM && !kval[ks]) v = f32x4{0.f, 0.f, 0.f, 0.f};
      epi_put(et, eoff<D>(16 * ks + li, 16 * ds + 4 * g), M::pack2(v[0] * osc, v[1] * osc),
              M::pack2(v[2] * osc, v[3] * osc));
    }
  }
  __syncthreads();  // orders the tile's writes before its reads
  epi_rows_out<T, D, KR>(et, lane, outp, ostr, kw, T_, DR);
}

// ============================================================================
// Launchers
// ============================================================================
// A head dim D runs in the kernels of layout width W (32, 64, 128 or 256: the
// LDS tiles, the fp16 Q copy and the loads take W columns, those past D read
// as zeros) whose MFMA loops cover DE columns, D rounded up to 32 (the
// columns DE .. W - 1 are zero and skipped). mfma_width and mfma_eff give W
// and DE; KAT_MFMA_WIDTHS lists the (W, DE) pairs that are built, each in a
// translation unit of its own (attn_mfma_w*.hip).
inline int mfma_width(int64_t D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }
inline int mfma_eff(int64_t D) {
  const int W = mfma_width(D);
  return W <= 64 ? W : (int)((D + 31) / 32 * 32);
}
#define KAT_MFMA_WIDTHS(X) \
  X(32, 32) X(64, 64) X(128, 96) X(128, 128) X(256, 160) X(256, 192) X(256, 224) X(256, 256)

// Backward workspace (each part 256-byte aligned): per-row stats (per 64-row
// tile two float[64]: 4 cinv, then -4 cinv Delta), the
// fp16 copy of Q ([B*H][T][D], D the layout width), per-tile Q exponents and dS-bound parts and
// dS exponents ([B*H][nt] each, nt = ceil(T / 64)), per-32-key K exponents,
// the dS^T tiles, and (banded calls only) one head's fp32 dQ partial sums.
// The dS^T region holds ds_cap() bytes of the call's mode's tiles (causal: the
// lower triangle of each head's 64 x 64 tiles, ~T^2 bytes per head; non-causal:
// all, ~2 T^2 bytes): as many heads as fit (a multiple of 8 when there are 8 or
// more, so that heads keep their XCD), and dK/dV + dQ run per group of heads.
// When one head's tiles exceed the cap, the head's key tiles split into bands
// of kQB-tile multiples (the widest whose first band fits the cap, at least
// kQB tiles = 512 keys) and dK/dV + dQ run per band of each head, dQ
// accumulating in fp32 in band order: the workspace stays within the cap plus
// O(B*H*T*D) bytes at every T (beyond T ~ 2^23 / cap-GiB^-1 the minimum band
// of 512 keys itself exceeds the cap). KAT_ATTN_DS_CAP_BYTES overrides the
// 4 GiB default (tests use it to run several groups or bands at small sizes).
inline size_t ds_cap() {
  const char* e = getenv("KAT_ATTN_DS_CAP_BYTES");
  const long long v = e ? atoll(e) : 0;
  return v > 0 ? (size_t)v : ((size_t)4 << 30);
}

inline BwdWs bwd_ws(void* base, int64_t B, int64_t H, int64_t T, int64_t D, bool causal) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const int64_t BH = B * H;
  const int nt = (int)((T + 63) / 64);
  const size_t rows = (size_t)(BH * T), tiles = (size_t)BH * (size_t)nt;
  const size_t cap = ds_cap();
  const size_t head = (size_t)ds_tiles_per_band(nt, causal, 0, nt) * 8192u;
  int64_t group = 1;
  int band = nt;
  size_t ds_bytes, acc_bytes = 0;
  if (head <= cap) {
    group = std::max<int64_t>(1, std::min<int64_t>(BH, (int64_t)(cap / head)));
    if (group >= 8) group &= ~(int64_t)7;
    ds_bytes = (size_t)group * head;
  } else {
    // the widest band (a multiple of kQB key tiles) whose tiles fit the cap;
    // the first band of a head is its largest
    int lo = 1, hi = (nt - 1) / kQB;  // in units of kQB tiles; hi * kQB < nt
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if ((size_t)ds_tiles_per_band(nt, causal, 0, mid * kQB) * 8192u <= cap)
        lo = mid;
      else
        hi = mid - 1;
    }
    band = std::max(1, lo) * kQB;
    ds_bytes = (size_t)ds_tiles_per_band(nt, causal, 0, band) * 8192u;
    acc_bytes = (size_t)nt * 64 * (size_t)D * sizeof(float);
  }
  char* p = reinterpret_cast<char*>(base);
  BwdWs w;
  size_t o = 0;
  auto take = [&](size_t n) { char* q = p + o; o += al(n); return q; };
  w.stats = reinterpret_cast<float*>(take(tiles * 128 * sizeof(float)));
  w.q16 = reinterpret_cast<f16*>(take(rows * (size_t)D * sizeof(f16)));
  w.qexp = reinterpret_cast<int*>(take(tiles * sizeof(int)));
  w.kexp = reinterpret_cast<int*>(take((size_t)BH * (size_t)((T + 31) / 32) * sizeof(int)));
  w.vnrm = reinterpret_cast<float*>(take(tiles * sizeof(float)));
  w.abnd = reinterpret_cast<float*>(take(tiles * sizeof(float)));
  w.bbnd = reinterpret_cast<float*>(take(tiles * sizeof(float)));
  w.ktile = reinterpret_cast<int*>(take(tiles * sizeof(int)));
  w.dst = reinterpret_cast<f16*>(take(ds_bytes));
  w.dqacc = acc_bytes ? reinterpret_cast<float*>(take(acc_bytes)) : nullptr;
  w.group = (int)group;
  w.band = band;
  w.bytes = o;
  return w;
}

template <typename T, int D, int DE, int MODE> int launch_fwd(const AttnArgs& a, hipStream_t st) {
  constexpr int QS = D == 256 ? 1 : kFwdQS, NW = D == 256 ? 8 : kNW, BMQ = NW * 16 * QS;
  const int64_t nb = (int64_t)((a.T + BMQ - 1) / BMQ) * a.B * a.H;
  hipLaunchKernelGGL((attn_fwd_k<T, D, MODE, QS, NW, DE>), dim3((unsigned)nb), dim3(64 * NW), 0, st, a);
  return check_launch("kat_attn_fwd (mfma)");
}

template <typename T, int D, int DE, int MODE>
int launch_bwd(const AttnArgs& a, void* ws, hipStream_t st) {
  constexpr bool kCausal = (MODE & kModeCausal) != 0;
  const BwdWs w = bwd_ws(ws, a.B, a.H, a.T, D, kCausal);
  const int BH = a.B * a.H;
  const int64_t tiles = (int64_t)BH * ((a.T + 63) / 64);
  // prep: the fp16 copy of Q, exponents, Delta and the row stats, the dS bound parts
  hipLaunchKernelGGL((attn_bwd_prep_k<T, D>), dim3((unsigned)tiles), dim3(256), 0, st, a, w);
  if (int rc = check_launch("kat_attn_bwd (prep)")) return rc;
  const int cpb = (a.T + 255) / 256;
  hipLaunchKernelGGL(attn_bwd_stscale_k<>, dim3((unsigned)((int64_t)BH * cpb)), dim3(256), 0, st, w, a.T, cpb);
  if (int rc = check_launch("kat_attn_bwd (stats scale)")) return rc;
  // per group of heads (and per band of key tiles): dK, dV (and the dS^T
  // tiles), then dQ from those tiles
  constexpr int KR = dkv_keys<D>(), BK = kNW * KR;  // keys per wave pair and per dK/dV block
  static_assert((kQB * 64) % BK == 0, "dK/dV blocks tile a band (bands start at multiples of kQB tiles)");
  constexpr int BQ = dq_block_queries<D>();                 // queries per dQ block
  const int nt = (a.T + 63) / 64, nqb = (a.T + BQ - 1) / BQ;
  for (int bh0 = 0; bh0 < BH; bh0 += w.group) {
    const int G = std::min(w.group, BH - bh0);
    for (int kb0 = 0; kb0 < nt; kb0 += w.band) {
      const int nk = std::min(w.band, nt - kb0);
      const int64_t nb = (std::min<int64_t>((int64_t)(kb0 + nk) * 64, a.T) - (int64_t)kb0 * 64 + BK - 1) / BK;
      // causal: the query blocks wholly before the band have no tiles in it
      const int64_t nbq = nqb - (kCausal ? (int64_t)kb0 * 64 / BQ : 0);
      hipLaunchKernelGGL((attn_bwd_dkv_k<T, D, MODE, KR, DE>), dim3((unsigned)(nb * G)), dim3(512), 0, st, a, w.stats,
                         w.q16, w.qexp, w.ktile, w.kexp, w.dst, bh0, G, kb0, nk);
      if (int rc = check_launch("kat_attn_bwd (dkv, mfma)")) return rc;
      hipLaunchKernelGGL((attn_bwd_dq_k<T, D, MODE, DE>), dim3((unsigned)(nbq * G)), dim3(64 * kDqW), 0, st, a,
                         w.kexp, w.ktile, w.dst, bh0, G, kb0, nk, w.dqacc);
      if (int rc = check_launch("kat_attn_bwd (dq, mfma)")) return rc;
    }
  }
  return 0;
}

// the kernel mode of a call: causal or not, with or without a padding mask
#define KAT_MODE_SWITCH(a, ...)                                                  \
  switch ((a.causal ? kModeCausal : 0) | (a.km != nullptr ? kModeKeyMask : 0)) { \
    case kModeCausal: { constexpr int MODE = kModeCausal; __VA_ARGS__; }         \
    case kModeCausal | kModeKeyMask: { constexpr int MODE = kModeCausal | kModeKeyMask; __VA_ARGS__; } \
    case kModeKeyMask: { constexpr int MODE = kModeKeyMask; __VA_ARGS__; }       \
    default: { constexpr int MODE = 0; __VA_ARGS__; }                            \
  }

template <typename T, int D, int DE> int attn_fwd_w(const AttnArgs& a, hipStream_t st) {
  KAT_MODE_SWITCH(a, return (launch_fwd<T, D, DE, MODE>(a, st)));
}
template <typename T, int D, int DE> int attn_bwd_w(const AttnArgs& a, void* ws, hipStream_t st) {
  KAT_MODE_SWITCH(a, return (launch_bwd<T, D, DE, MODE>(a, ws, st)));
}

// instantiated in the width translation units
#define KAT_MFMA_EXTERN(W, E)                                                              \
  extern template int attn_fwd_w<bf16, W, E>(const AttnArgs&, hipStream_t);              \
  extern template int attn_fwd_w<f16, W, E>(const AttnArgs&, hipStream_t);               \
  extern template int attn_bwd_w<bf16, W, E>(const AttnArgs&, void*, hipStream_t);       \
  extern template int attn_bwd_w<f16, W, E>(const AttnArgs&, void*, hipStream_t);
#define KAT_MFMA_INSTANTIATE(W, E)                                                         \
  template int attn_fwd_w<bf16, W, E>(const AttnArgs&, hipStream_t);                     \
  template int attn_fwd_w<f16, W, E>(const AttnArgs&, hipStream_t);                      \
  template int attn_bwd_w<bf16, W, E>(const AttnArgs&, void*, hipStream_t);              \
  template int attn_bwd_w<f16, W, E>(const AttnArgs&, void*, hipStream_t);

}  // namespace kat
