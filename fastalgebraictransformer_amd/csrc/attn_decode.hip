// Single-query rational attention over a KV cache (decode) on gfx950.
//
// The reference's generate() re-runs the whole forward over the prefix for
// every new token (algebraic_model.py:239-265), i.e. a causal attention whose
// last row is the only one that changes. This computes that last row directly
// from cached K / V:
//   i = n - 1 (the newest cached key is the query's own position),
//   s_j = scale q.k_j - slope (i - j),  f_j = sigma(s_j)^4   (j < n)
//   L = sum_j f_j,  o = sum_j f_j v_j / (L + eps)            (forward.py:110-159)
//
// Design (MI355X): the work is a GEMV over K and V, so HBM bandwidth bounds it
// (4 D bytes per cached key in bf16). One (batch, head) pair has too few keys
// to fill 256 CUs, so the keys are split into chunks, one work-group each,
// with 16-byte lanes spread across a key row and several rows per lane in
// flight. sigma^4 lies in (0, 1), so the attention needs no running maximum:
// each chunk writes the plain partial sums (sum f v, sum f), and a second
// kernel adds the chunks in a fixed order (deterministic) and normalises.

#include <algorithm>
#include <mutex>

#include "kat_common.h"
#include "kat_internal.h"

namespace kat {

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* L;                // [B*H] fp32, or nullptr
  const float* slopes;     // [H]
  const int32_t* lengths;  // [B] keys cached per batch row, or nullptr (all T)
  int B, H, T, D;          // T: rows addressable per (b, h) in the cache
  int64_t sq[2], sk[3], sv[3], so[2];
  float scale, eps;
  int splits, chunk;       // chunk: keys per work-group
};

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecInFlight = 4;  // rows per lane in flight
constexpr int kDecCombThreads = 256;  // combine: one thread per column and one for the row sums

template <typename T, int D> struct DecShape {
  static constexpr int EPL = 16 / (int)sizeof(T);  // elements per lane (one 16-byte load)
  static constexpr int LPR = D / EPL;              // lanes per key row
  static constexpr int RPW = 64 / LPR;             // rows per wave per pass
  static constexpr int RPP = RPW * kDecWaves;      // rows per block per pass
  static_assert(D % EPL == 0 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "row layout");
};

// one cached key or value row piece (16 bytes). Each cache row is read once per
// call, so the loads are non-temporal: at B=16 (512 MB of cache) a call took
// 84.7 instead of 97.8 us, at B=4, n=32768 172.7 instead of 195.1 us.
template <typename T, int EPL>
__device__ __forceinline__ VecT<T, EPL> ld_row_nt(const T* p) {
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  static_assert(sizeof(VecT<T, EPL>) == 16, "16-byte pieces");
  return __builtin_bit_cast(VecT<T, EPL>, __builtin_nontemporal_load(reinterpret_cast<const i32x4_t*>(p)));
}

// partials: part[(bh * splits + split) * (D + 1) + d] = sum_j f_j v_j[d], [.. + D] = sum_j f_j.
// D is the layout width; a head dim a.D below it leaves the lanes past a.D
// with a zero query (so they add nothing to the scores) and their columns'
// partials unused (the combine stores a.D columns). Those lanes read the
// row's first columns, so that no load leaves the row.
template <typename T, int D>
__global__ __launch_bounds__(kDecThreads) void attn_decode_part_k(DecodeArgs a, float* __restrict__ part) {
  typedef DecShape<T, D> S;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPW = S::RPW, RPP = S::RPP, U = kDecInFlight;
  __shared__ float sh_acc[kDecWaves][D];
  __shared__ float sh_l[kDecWaves];
  const int bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sub = lane % LPR, grp = lane / LPR;
  int n = a.lengths ? a.lengths[b] : a.T;
  n = min(max(n, 0), a.T);  // a bad length cannot move a read out of the cache
  const int j0 = split * a.chunk, j1 = min(j0 + a.chunk, n);
  const float ipos = (float)(n - 1);  // the query's position
  const float slope = a.slopes[h];

  const bool din = sub * EPL < a.D;
  const int col0 = din ? sub * EPL : 0;
  float qv[EPL];
  load_acc<T, EPL>((const T*)a.q + b * a.sq[0] + h * a.sq[1] + col0, qv);
#pragma unroll
  for (int e = 0; e < EPL; ++e) qv[e] = din ? qv[e] * a.scale : 0.f;
  const T* kp = (const T*)a.k + b * a.sk[0] + h * a.sk[1] + col0;
  const T* vp = (const T*)a.v + b * a.sv[0] + h * a.sv[1] + col0;

  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  float l = 0.f;
  // wave-uniform loop; lane group `grp` takes row base + u RPP + grp
  for (int base = j0 + w * RPW; base < j1; base += RPP * U) {
    VecT<T, EPL> kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(base + u * RPP + grp, j1 - 1);  // rows past the chunk re-read its last
      kr[u] = ld_row_nt<T, EPL>(kp + (int64_t)j * a.sk[2]);
      vr[u] = ld_row_nt<T, EPL>(vp + (int64_t)j * a.sv[2]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = base + u * RPP + grp;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d = fmaf(qv[e], to_acc(kr[u].v[e]), d);
#pragma unroll
      for (int off = 1; off < LPR; off <<= 1) d += __shfl_xor(d, off, 64);
      const float s = d - slope * (ipos - (float)j);  // forward.py:129-133
      const float sg = rsig(s);                        // forward.py:137-140
      const float s2 = sg * sg;
      const float f = j < j1 ? s2 * s2 : 0.f;
      l += f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = fmaf(f, to_acc(vr[u].v[e]), acc[e]);
    }
  }
  // lanes with the same `sub` hold the same columns: add across the row groups
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
    l += __shfl_xor(l, off, 64);
  }
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) sh_acc[w][sub * EPL + e] = acc[e];
    if (sub == 0) sh_l[w] = l;
  }
  __syncthreads();
  float* out = part + ((int64_t)bh * a.splits + split) * (D + 1);
  for (int d = threadIdx.x; d <= D; d += kDecThreads) {
    float t = 0.f;
#pragma unroll
    for (int ww = 0; ww < kDecWaves; ++ww) t += d < D ? sh_acc[ww][d] : sh_l[ww];
    out[d] = t;
  }
}

// o = sum_s acc_s / (sum_s l_s + eps), L = sum_s l_s; one block per (b, h).
// Thread d < D sums column d and thread D the row sums l, all at once: the
// partials come from work-groups on other XCDs (other L2s), so every load is
// a round trip to memory, and each thread keeps eight independent loads in
// flight (eight running sums over the splits s = 8 i + r, added in a fixed
// order: deterministic).
template <typename T, int D>
__device__ __forceinline__ float sum_splits(const float* __restrict__ p, int S, int col) {
  float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int s = 0;
  for (; s + 8 <= S; s += 8) {
#pragma unroll
    for (int r = 0; r < 8; ++r) t[r] += p[(int64_t)(s + r) * (D + 1) + col];
  }
#pragma unroll
  for (int r = 0; r < 7; ++r)
    if (s + r < S) t[r] += p[(int64_t)(s + r) * (D + 1) + col];
  return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

template <typename T, int D>
__global__ __launch_bounds__(kDecCombThreads) void attn_decode_combine_k(DecodeArgs a, const float* __restrict__ part) {
  __shared__ float sh_inv;
  const int bh = blockIdx.x, b = bh / a.H, h = bh - b * a.H;
  const float* p = part + (int64_t)bh * a.splits * (D + 1);
  float t[(D + kDecCombThreads) / kDecCombThreads];  // columns threadIdx.x + k * threads
#pragma unroll
  for (int k = 0; k < (D + kDecCombThreads) / kDecCombThreads; ++k) {
    const int col = (int)threadIdx.x + k * kDecCombThreads;
    t[k] = col <= D ? sum_splits<T, D>(p, a.splits, col) : 0.f;
    if (col == D) {
      if (a.L) a.L[bh] = t[k];
      sh_inv = 1.f / (t[k] + a.eps);  // forward.py:150
    }
  }
  __syncthreads();
  const float inv = sh_inv;
  T* o = (T*)a.o + b * a.so[0] + h * a.so[1];
#pragma unroll
  for (int k = 0; k < (D + kDecCombThreads) / kDecCombThreads; ++k) {
    const int col = (int)threadIdx.x + k * kDecCombThreads;
    if (col < a.D) o[col] = from_acc<T>(t[k] * inv);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Work-groups: enough chunks that B*H*splits covers the CUs twice, no chunk
// smaller than one block pass.
static void decode_split(int64_t B, int64_t H, int64_t T, int rpp, int& splits, int& chunk) {
  const int64_t want = (2 * (int64_t)num_cus() + B * H - 1) / std::max<int64_t>(1, B * H);
  const int64_t max_splits = std::max<int64_t>(1, (T + rpp - 1) / rpp);
  const int64_t s = std::max<int64_t>(1, std::min(want, max_splits));
  int64_t c = (T + s - 1) / s;
  c = (c + rpp - 1) / rpp * rpp;
  splits = (int)std::max<int64_t>(1, (T + c - 1) / c);
  chunk = (int)c;
}

// the kernels' layout width for a head dim: 64, 128 or 256 (16-bit types; any
// multiple of 8 up to 256) or 32, 64 or 128 (fp32; multiples of 4 up to 128);
// 0 if none serves
static int decode_layout(int64_t D, int dtype) {
  if (dtype == KAT_F32) return D < 4 || D > 128 || D % 4 ? 0 : D <= 32 ? 32 : D <= 64 ? 64 : 128;
  if (dtype == KAT_BF16 || dtype == KAT_F16) return D < 8 || D > 256 || D % 8 ? 0 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
  return 0;
}

static int decode_rpp(int D, int dtype) {
  const int epl = 16 / dtype_size(dtype);
  return (64 / (decode_layout(D, dtype) / epl)) * kDecWaves;
}

static bool decode_supported(int64_t D, int dtype) { return decode_layout(D, dtype) != 0; }

template <typename T, int D> static int launch_decode(const DecodeArgs& a, float* part, hipStream_t st) {
  hipLaunchKernelGGL((attn_decode_part_k<T, D>), dim3((unsigned)a.splits, (unsigned)(a.B * a.H)),
                     dim3(kDecThreads), 0, st, a, part);
  if (int rc = check_launch("kat_attn_decode (partials)")) return rc;
  hipLaunchKernelGGL((attn_decode_combine_k<T, D>), dim3((unsigned)(a.B * a.H)), dim3(kDecCombThreads), 0, st, a,
                     (const float*)part);
  return check_launch("kat_attn_decode (combine)");
}

template <typename T> static int decode_d(const DecodeArgs& a, float* part, hipStream_t st) {
  switch (decode_layout(a.D, sizeof(T) == 4 ? KAT_F32 : KAT_BF16)) {
    case 32: if constexpr (sizeof(T) == 4) return launch_decode<T, 32>(a, part, st); break;
    case 64: return launch_decode<T, 64>(a, part, st);
    case 128: return launch_decode<T, 128>(a, part, st);
    case 256: if constexpr (sizeof(T) == 2) return launch_decode<T, 256>(a, part, st); break;
  }
  return fail(KAT_EUNSUPPORTED, "kat_attn_decode: head dim %d", a.D);
}

}  // namespace kat

using namespace kat;

extern "C" size_t kat_attn_decode_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D,
                                                 int dtype) {
  if (B <= 0 || H <= 0 || T <= 0 || !decode_supported(D, dtype)) return 0;
  int splits, chunk;
  decode_split(B, H, T, decode_rpp((int)D, dtype), splits, chunk);
  return (size_t)(B * H) * (size_t)splits * (size_t)(decode_layout(D, dtype) + 1) * sizeof(float);
}

// Argument checks and launch shared by kat_attn_decode and
// kat_attn_decode_noalloc. get_part(need, rc) returns the partials buffer for
// `need` bytes, or nullptr after recording an error and setting rc to its code.
template <typename GetPart>
static int decode_impl(const char* nm, const void* q, const void* k, const void* v, void* out, float* L,
                       const float* slopes, const int32_t* lengths, int64_t B, int64_t H, int64_t T,
                       int64_t D, const int64_t* strides, float scale, float eps, int dtype, void* stream,
                       GetPart get_part) {
  if (B < 0 || H < 0 || T < 0 || D < 0) return fail(KAT_EINVAL, "%s: negative size", nm);
  if (B * H > 0xffffLL * 0x7fffLL || T > 0x3fffffffLL)
    return fail(KAT_EUNSUPPORTED, "%s: B*H or T too large", nm);
  if (!decode_supported(D, dtype))
    return fail(KAT_EUNSUPPORTED, "%s: head dim %lld with dtype %d", nm, (long long)D, dtype);
  if (B * H == 0) return KAT_OK;
  if (!q || !k || !v || !out || !slopes || !strides) return fail(KAT_EINVAL, "%s: null pointer", nm);
  const int esz = dtype_size(dtype);
  // 16-byte rows: q and out per (b, h); k and v per (b, h, t)
  const int64_t* s = strides;
  for (int t = 0; t < 10; ++t)
    if ((s[t] * esz) % 16 != 0) return fail(KAT_EUNSUPPORTED, "%s: strides must keep rows 16-byte aligned", nm);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(KAT_EUNSUPPORTED, "%s: tensors must be 16-byte aligned", nm);
  if (T > 0 && (s[4] < D || s[7] < D))
    return fail(KAT_EINVAL, "%s: cache row stride < D", nm);
  DecodeArgs a = {};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.L = L;
  a.slopes = slopes;
  a.lengths = lengths;
  a.B = (int)B;
  a.H = (int)H;
  a.T = (int)T;
  a.D = (int)D;
  a.sq[0] = s[0]; a.sq[1] = s[1];
  a.sk[0] = s[2]; a.sk[1] = s[3]; a.sk[2] = s[4];
  a.sv[0] = s[5]; a.sv[1] = s[6]; a.sv[2] = s[7];
  a.so[0] = s[8]; a.so[1] = s[9];
  a.scale = scale;
  a.eps = eps;
  decode_split(B, H, std::max<int64_t>(T, 1), decode_rpp((int)D, dtype), a.splits, a.chunk);
  const size_t need = (size_t)(B * H) * (size_t)a.splits * (size_t)(decode_layout(D, dtype) + 1) * sizeof(float);
  int rc = KAT_OK;
  float* part = get_part(need, rc);
  if (!part) return rc;  // get_part recorded the message
  const hipStream_t st = as_stream(stream);
  switch (dtype) {
    case KAT_F32: return decode_d<float>(a, part, st);
    case KAT_BF16: return decode_d<bf16>(a, part, st);
    case KAT_F16: return decode_d<f16>(a, part, st);
  }
  return fail(KAT_EUNSUPPORTED, "%s: unsupported dtype %d", nm, dtype);
}

extern "C" int kat_attn_decode(const void* q, const void* k, const void* v, void* out, float* L,
                               const float* slopes, const int32_t* lengths, void* workspace,
                               size_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                               const int64_t* strides, float scale, float eps, int dtype,
                               void* stream) {
  const char* nm = "kat_attn_decode";
  return decode_impl(nm, q, k, v, out, L, slopes, lengths, B, H, T, D, strides, scale, eps, dtype,
                     stream, [&](size_t need, int& rc) -> float* {
                       if (!workspace || workspace_bytes < need) {
                         rc = fail(KAT_EINVAL, "%s: workspace %zu bytes < required %zu", nm, workspace_bytes,
                                   need);
                         return nullptr;
                       }
                       return reinterpret_cast<float*>(workspace);
                     });
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the partials live in a fixed device array of the
// library (one copy per GPU, held until the process ends) instead of a
// caller's workspace. `scratch` names a host-side stand-in; its device
// address on the current GPU comes from hipGetSymbolAddress, looked up once
// per device on the first call and kept.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[KAT_DECODE_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// device address of `scratch` on the current device, or nullptr (error
// recorded, rc set to its code)
float* device_scratch(const char* nm, int& rc) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    rc = fail(KAT_EHIP, "%s: no current HIP device", nm);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      rc = fail(KAT_EHIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", nm, dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int kat_attn_decode_noalloc(const void* q, const void* k, const void* v, void* out, float* L,
                                       const float* slopes, const int32_t* lengths, int64_t B, int64_t H,
                                       int64_t T, int64_t D, const int64_t* strides, float scale,
                                       float eps, int dtype, void* stream) {
  const char* nm = "kat_attn_decode_noalloc";
  return decode_impl(nm, q, k, v, out, L, slopes, lengths, B, H, T, D, strides, scale, eps, dtype,
                     stream, [&](size_t need, int& rc) -> float* {
                       if (need > (size_t)KAT_DECODE_SCRATCH_BYTES) {
                         rc = fail(KAT_EUNSUPPORTED,
                              "%s: the partials need %zu bytes, more than the %zu-byte scratch array "
                              "(B*H*splits*(D+1) floats; use kat_attn_decode with a workspace)",
                              nm, need, (size_t)KAT_DECODE_SCRATCH_BYTES);
                         return nullptr;
                       }
                       return device_scratch(nm, rc);
                     });
}
