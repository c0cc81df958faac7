// Device building blocks of the gfx950 (CDNA4) MFMA attention kernels:
// MFMA wrappers, LDS fragment reads, LDS-DMA tile staging, block ordering.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "kat_common.h"

namespace kat {
namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// v_mfma_f32_16x16x32_{bf16,f16}. Operand layout (lane l, g = l / 16, li = l % 16):
// A[m = li][k-set g], B[k-set g][n = li], C[4 g + j][li] (j = 0..3). A and B only
// have to agree on which 8 k-indices form k-set g.
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  static __device__ __forceinline__ f32x4 mma(const i16x8& a, const i16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8)a, (bf16x8)b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x, y}), bf16x2));
  }
};
template <> struct Mfma<f16> {
  static __device__ __forceinline__ f32x4 mma(const i16x8& a, const i16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16((f16x8)a, (f16x8)b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x, y}), f16x2));
  }
};

// fp16 operands for the dS products: dS = p g (dP - Delta) is rounded to fp16
// (11-bit significand) rather than bf16 before dQ = dS K and dK = dS^T Q, so its
// rounding error is 4x smaller. K and Q enter those products (and S itself) as
// fp16 copies; bf16 -> fp16 is exact for |x| in [2^-14, 65504], magnitudes
// above 65504 are clamped and smaller ones keep fp16's subnormal spacing 2^-24.
__device__ __forceinline__ f32x4 mma_f16(const i16x8& a, const i16x8& b, const f32x4& c) {
  return Mfma<f16>::mma(a, b, c);
}
__device__ __forceinline__ uint32_t pack2_f16(float x, float y) { return Mfma<f16>::pack2(x, y); }

template <typename T> __device__ __forceinline__ i16x8 to_f16x8(const i16x8& v);
template <> __device__ __forceinline__ i16x8 to_f16x8<f16>(const i16x8& v) { return v; }
template <> __device__ __forceinline__ i16x8 to_f16x8<bf16>(const i16x8& v) {
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

// fp16 copy of 8 elements of T multiplied by f (a power of two chosen by
// tile_exp, so the product is exact); clamped to +-65504 as a guard.
template <typename T> __device__ __forceinline__ i16x8 to_f16x8s(const i16x8& v, float f) {
  const VecT<T, 8> x = __builtin_bit_cast(VecT<T, 8>, v);
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = (float)x.v[2 * e] * f, hi = (float)x.v[2 * e + 1] * f;
    o[e] = pack2_f16(fminf(fmaxf(lo, -65504.f), 65504.f), fminf(fmaxf(hi, -65504.f), 65504.f));
  }
  return __builtin_bit_cast(i16x8, o);
}

// largest |element| of 8 elements of T
template <typename T> __device__ __forceinline__ float absmax8(const i16x8& v) {
  const VecT<T, 8> x = __builtin_bit_cast(VecT<T, 8>, v);
  float m = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)x.v[e]));
  return m;
}

// Power-of-two exponent for the fp16 copy of a 64-row tile whose largest
// magnitude is m. bf16 -> fp16 is exact for magnitudes in [2^-14, 65504]; a
// tile with m in [2^-6, 2^15) is copied unscaled (its elements below 2^-14
// are then at least 2^-8 below m, where fp16's subnormal spacing 2^-24 is
// far below bf16's own rounding of m), any other tile is scaled so that
// m 2^e lies in [2^14, 2^15). e is clamped to [-40, 40], which covers tiles
// with m in [2^-46, 2^55]; zero and non-finite m give 0.
__device__ __forceinline__ int tile_exp(float m) {
  if (m >= 0x1p-6f && m < 0x1p15f) return 0;
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 0;
  int E;
  (void)frexpf(m, &E);  // m = f 2^E, f in [0.5, 1)
  return std::min(40, std::max(-40, 15 - E));
}

// Power-of-two exponent k for an fp16 operand whose magnitudes are bounded by
// b: b 2^k lies in [2^13, 2^14), a quarter of fp16's range, so that values
// reach fp16's subnormal range only 27 binades below the bound. Clamped to
// [-100, 100]; zero or non-finite b gives 0.
__device__ __forceinline__ int ds_exp(float b) {
  if (!(b > 0.f) || !(b <= 3.4e38f)) return 0;
  int E;
  (void)frexpf(b, &E);
  return std::min(100, std::max(-100, 14 - E));
}

// Index of the calling wave in its block as a wave-uniform (scalar) value.
// threadIdx.x >> 6 is the same in every lane of a wave, but the compiler
// cannot prove it, and branches on values derived from it become exec-mask
// saves and restores around every role and tile condition; read from the first
// lane they are plain scalar branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ i16x8 pack_frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(i16x8, (u32x4{a, b, c, d}));
}

// ---------------------------------------------------------------------------
// Buffer resources. Loads through a raw buffer resource (stride 0) return zero
// for bytes at or beyond num_records, which zero-fills rows past the sequence
// end without branches.
// ---------------------------------------------------------------------------
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format
// A buffer offset at or past every resource's num_records (the kernels keep
// extents below 2^31): the load returns zeros. The columns a tile or fragment
// holds beyond the head dim of a call (kernels built for a wider layout, e.g.
// D = 96 in the D = 128 kernels) take it, so they read as zeros.
constexpr uint32_t kOobOff = 0x80000000u;
__device__ __forceinline__ uint32_t col_off(uint32_t off, int col, int cols) { return col < cols ? off : kOobOff; }

// resource for kernel-side loads through the compiler builtin
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ i16x8 load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(i16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// resource as four SGPRs, for the LDS-DMA below
__device__ __forceinline__ i32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = kRsrcWord3;
  return r;
}

// LDS-DMA: every active lane l copies 16 bytes at buffer offset voff into LDS at
// lds + 16 l (buffer_load_dwordx4 ... lds, M0 = LDS base). Issued through inline
// asm so that the compiler adds no wait for it before unrelated LDS reads; the
// kernel waits with dma_wait() before the barrier that publishes the tile.
// dma_wait() is the s_waitcnt builtin (vmcnt(0), expcnt and lgkmcnt left at
// their maxima: 0x0F70 in the gfx9 encoding) rather than asm, so the compiler's
// wait tracking also sees every earlier vector-memory load as complete.
// The LDS destination is a 32-bit LDS address (lds_addr of a __shared__ array
// plus a wave-uniform offset), so that it stays in SGPRs.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}
// NT: the non-temporal cache policy, for data read once (it is then evicted
// first from L2 and does not displace tiles other blocks re-read).
template <bool NT = false>
__device__ __forceinline__ void dma16(const i32x4& r, uint32_t lds, uint32_t voff) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(lds);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(la), "v"(voff),
                 "s"(r)
                 : "memory");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(la), "v"(voff),
                 "s"(r)
                 : "memory");
}
__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---------------------------------------------------------------------------
// LDS tiles: rows of D 16-bit elements with the 16-byte chunks of row r XOR-ed
// by swz(r), a GF(2)-linear map of the row's low 4 bits (listed by the images of
// bits 0..3). LDS has 64 banks of 4 bytes; ds_read_b64_tr_b16 serves 32
// consecutive lanes per pass, and ds_read_b128 serves 16 lanes per pass grouped
// by (lane bit 5, parity of lane bits 2..4) -- a model fitted to timings of 48
// swizzles on gfx950. Under it these maps leave both reads conflict-free: the
// row fragments (rows r0 + lane % 16, chunk lane / 16 (+ const)) and the
// transposed fragments (rows r0 + 4 (lane / 16) + lane % 16 / 4, two chunks).
// D = 32 (rows of 4 chunks, 64 bytes: rows four apart share banks): images
// 0, 0, 2, 1, so the four rows of a bank group take four different chunks in
// the row reads, and rows 0-3 and 4-7 take disjoint chunk pairs in the
// transposed reads.
// ---------------------------------------------------------------------------
// D = 256 and 512 (rows of 512 / 1024 bytes: a chunk's bank depends only on
// its index mod 16, as for D = 128; 512 16-bit units are the fp32 kernels'
// rows of 256 floats) take the D = 128 map on the low 4 chunk bits.
template <int D> __device__ __forceinline__ int swz(int row) {
  static_assert(D == 32 || D == 64 || D == 128 || D == 256 || D == 512,
                "swizzle defined for D = 32, 64, 128, 256, 512");
  constexpr bool W = D >= 128;
  constexpr int i0 = W ? 8 : D == 64 ? 1 : 0, i1 = W ? 3 : D == 64 ? 2 : 0,
                i2 = W ? 5 : D == 64 ? 4 : 2, i3 = W ? 11 : D == 64 ? 5 : 1;
  return ((row & 1) ? i0 : 0) ^ ((row & 2) ? i1 : 0) ^ ((row & 4) ? i2 : 0) ^ ((row & 8) ? i3 : 0);
}
template <int D> __device__ __forceinline__ int soff(int row, int col) {
  return row * D + (((col >> 3) ^ swz<D>(row)) << 3) + (col & 7);
}

__device__ __forceinline__ i16x8 lds16(const short* p) { return *reinterpret_cast<const i16x8*>(p); }

// 16-byte non-temporal global load (data read once)
template <typename T> __device__ __forceinline__ i16x8 ld_nt16(const T* p) {
  return __builtin_bit_cast(i16x8, __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p)));
}

// Transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, result
// lane i element j is element i % 4 of the 8 bytes addressed by lane i / 4 + 4 j.
__device__ __forceinline__ i16x4 lds_tr(const short* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// A-operand fragment of a row-major swizzled tile read transposed: lane (g, li)
// gets column c0 + li of rows r0 + 4 g + {0..3} (elements 0-3) and
// r0 + 16 + 4 g + {0..3} (elements 4-7).
template <int D>
__device__ __forceinline__ i16x8 frag_tr(const short* tile, int r0, int c0, int g, int li) {
  const int row = r0 + 4 * g + (li >> 2), col = c0 + 4 * (li & 3);
  const i16x4 lo = lds_tr(tile + soff<D>(row, col));
  const i16x4 hi = lds_tr(tile + soff<D>(row + 16, col));
  return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Stage a ROWS-row tile (rows row0 .. row0 + ROWS - 1 of a [rows][stride]
// matrix, D columns) into a swizzled LDS tile with the NW waves of the block:
// each wave issues ROWS / RPS / NW DMA segments of RPS rows.
template <int D, int NW, int ROWS = 64> struct TileDma {
  static constexpr int CPR = D / 8;             // 16-byte chunks per row
  static constexpr int RPS = 64 / CPR;          // rows per 1 KB segment
  static constexpr int SEGS = ROWS / RPS / NW;  // segments per wave
  static_assert(SEGS >= 1 && SEGS * RPS * NW == ROWS, "tile rows must split evenly over the waves");
  uint32_t off[SEGS];
  // cols: the matrix's columns (<= D); chunks past them load zeros
  __device__ __forceinline__ void init(int w, int lane, uint32_t stride, int cols = D) {
#pragma unroll
    for (int u = 0; u < SEGS; ++u) {
      const int row = (w * SEGS + u) * RPS + lane / CPR;
      const int c = (lane % CPR) ^ swz<D>(row);
      off[u] = col_off((row * stride + 8 * c) * 2, 8 * c, cols);
    }
  }
  // base: first row of the matrix; bytes: its extent; row0: first tile row
  template <bool NT = false>
  __device__ __forceinline__ void issue(short* tile, const void* base, uint32_t bytes, int row0,
                                        uint32_t stride, int w) const {
    const uint32_t skip = (uint32_t)row0 * stride * 2;
    const i32x4 r = rsrc_words((const char*)base + skip, bytes > skip ? bytes - skip : 0u);
    const uint32_t l0 = lds_addr(tile) + (uint32_t)(__builtin_amdgcn_readfirstlane(w) * SEGS * RPS * D * 2);
#pragma unroll
    for (int u = 0; u < SEGS; ++u) dma16<NT>(r, l0 + (uint32_t)(u * RPS * D * 2), off[u]);
  }
};

// Block order. Workgroups are dispatched round-robin over the 8 XCDs (block id
// i runs on XCD i % 8), and each XCD has its own L2. Heads are assigned to XCDs
// (head h on XCD h % 8 when B*H is a multiple of 8) and each XCD takes the
// tiles of its heads longest (most causal work) first across all its heads,
// which balances the causal triangle over the XCD's CUs.
// Returns the (b*H + h) index and the tile rank (0 = most work).
__device__ __forceinline__ void block_order(int id, int BH, int& bh, int& rank) {
  if ((BH & 7) == 0) {
    const int xcd = id & 7, slot = id >> 3, hpx = BH >> 3;
    rank = slot / hpx;
    bh = xcd + 8 * (slot - rank * hpx);
  } else {
    rank = id / BH;
    bh = id - rank * BH;
  }
}

// Epilogue staging: a wave's output rows (R rows of D 16-bit elements) pass
// through a row-major LDS tile so that the global stores write whole rows (a
// 16-byte piece per lane, D / 8 lanes per row) instead of the 8-byte pieces of
// the MFMA C layout, which leave every store instruction 32-byte fragments of
// 16 rows. The tile's 16-byte chunks are XOR-ed by the row's low bits, so the
// 8-byte writes of 16 consecutive rows and the 16-byte reads spread over the
// banks.
template <int D> __device__ __forceinline__ int eoff(int row, int col) {
  return row * D + ((((col >> 3) ^ row) & (D / 8 - 1)) << 3) + (col & 7);
}
// element (row, col .. col + 3) of the staging tile: 4 values packed as 2 x 2
__device__ __forceinline__ void epi_put(short* tile, int off, uint32_t lo, uint32_t hi) {
  *reinterpret_cast<u32x2*>(tile + off) = u32x2{lo, hi};
}
// rows 0 .. R - 1 of the tile to base[(row0 + r) * stride], rows with
// row0 + r >= nrows and columns at or past cols skipped; the tile must be complete (written by this wave,
// with a barrier or an LDS wait in between). Non-temporal stores: the outputs
// are not re-read by the kernel that writes them, and write-back stores left
// their lines in L2 where the still-running blocks keep their K / V, Q16 / dO
// and K16 tiles (measured: backward 2.6% slower at config 3, 1.2% at config 5's
// shape, forward 0.5%).
template <typename T, int D, int R>
__device__ __forceinline__ void epi_rows_out(const short* tile, int lane, T* __restrict__ base, int64_t stride,
                                             int row0, int nrows, int cols = D) {
  constexpr int CPR = D / 8, RPI = 64 / CPR;  // chunks per row, rows per instruction
#pragma unroll
  for (int i = 0; i < R / RPI; ++i) {
    const int r = i * RPI + lane / CPR, c = lane % CPR;
    const i16x8 v = *reinterpret_cast<const i16x8*>(tile + eoff<D>(r, 8 * c));
    if (row0 + r < nrows && 8 * c < cols)
      __builtin_nontemporal_store(v, reinterpret_cast<i16x8*>(base + (int64_t)(row0 + r) * stride + 8 * c));
  }
}

// extent in bytes of T rows of D 16-bit elements at a row stride (elements);
// D: the matrix's own columns
__device__ __forceinline__ uint32_t row_bytes(int T, uint32_t stride, int D) {
  return ((uint32_t)(T - 1) * stride + (uint32_t)D) * 2u;
}

}  // namespace mfma
}  // namespace kat
