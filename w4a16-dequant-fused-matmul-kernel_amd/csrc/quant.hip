// Quantise / pack / unpack / dequantise kernels, bit-exact with the reference's
// PyTorch quantiser as torch evaluates it on the CPU
// (w4a16-kernel/src/w4a16/quant.py:45-178):
//   scale = (gmax - gmin) / 15        IEEE fp32 division (not a reciprocal multiply)
//   scale = scale > 0 ? scale : 1
//   zero  = clamp(rint(-gmin / scale), 0, 15)   compare-select clamp, -0.0 survives
//   q     = clamp(rint(W / scale) + zero, 0, 15) with the fp32 scale
//   scales, zeros -> fp16 (RNE); codes packed 8 per int32, row 8i+j in nibble j.
// rint is round-half-to-even (v_rndne_f32).  HIP divides fp32 with the correctly
// rounded sequence by default, and the build never enables fast-math, so the
// compare-selects are not folded into min/max (which could drop -0.0).
// Group minimum, as torch's CPU amin(dim=1) returns it when a group's minimum
// is a zero and the group holds both +0.0 and -0.0 (measured on torch's CPU
// reduction; the same on its DEFAULT, AVX2 and AVX512 code paths):
//  * N >= 2 (the reduced rows are strided): columns in whole blocks of 32
//    (n < 32 * (N / 32), the vectorised outer reduction) take the last zero in
//    k order (v <= min ? v : min), the N % 32 tail columns (its scalar loop) the
//    first (v < min ? v : min);
//  * N == 1 (the group's G values are contiguous): G < 32 takes the first zero;
//    G >= 32 follows the vectorised inner reduction (inner_zero_min below).
// Only the sign of the zero-point depends on it; the group maximum's zero sign
// reaches no output (gmax - gmin is the same for either zero, or the scale is
// replaced by 1).
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

// Input element traits: fp16 weights arrive as raw bits, fp32 as floats.
struct InF16 {
  typedef uint16_t T;
  static __device__ __forceinline__ float val(T b) { return (float)as_h(b); }
  static __device__ __forceinline__ bool nonfinite(T b) { return (b & 0x7C00u) == 0x7C00u; }
  // four consecutive elements (8-byte aligned)
  static __device__ __forceinline__ void load4(const T* p, T out[4]) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = v.x & 0xFFFFu;
    out[1] = v.x >> 16;
    out[2] = v.y & 0xFFFFu;
    out[3] = v.y >> 16;
  }
};
struct InF32 {
  typedef float T;
  static __device__ __forceinline__ float val(T v) { return v; }
  static __device__ __forceinline__ bool nonfinite(T v) {
    return (__builtin_bit_cast(uint32_t, v) & 0x7F800000u) == 0x7F800000u;
  }
  // four consecutive elements (16-byte aligned)
  static __device__ __forceinline__ void load4(const T* p, T out[4]) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
};

// Running group minimum; tie_last selects which of two equal values (only
// +0.0 / -0.0 differ in bits) is kept.
__device__ __forceinline__ float min_step(float v, float mn, bool tie_last) {
  return (v < mn || (tie_last && v == mn)) ? v : mn;
}

// N == 1, G >= 32, a group whose minimum is a zero: the zero torch's
// vectorised inner reduction returns.  It reduces the first 32 * (G / 32) values
// with 4 accumulators of 8 lanes (position p in lane p % 8 of accumulator
// (p / 8) % 4; a tie keeps the later value), folds accumulator 0 with 1, 2, 3 in
// turn (a tie keeps the later accumulator) and the lanes toward lane 0 (a tie
// keeps the lower lane), then scans the G % 32 tail values (a tie keeps the
// running minimum).  So among the zeros the lowest lane wins, then the highest
// accumulator, then the latest position; a tail zero only wins when no zero
// precedes the tail, and then the first one.  Only called when the group's
// minimum is a zero, so it rescans just those groups.
template <class IN>
__device__ float inner_zero_min(const typename IN::T* __restrict__ src, int G) {
  const int B = 32 * (G / 32);
  uint64_t best = ~0ull;
  float z = 0.0f;
  for (int p = 0; p < G; ++p) {
    const float v = IN::val(src[p]);
    if (v != 0.0f) continue;
    const int s = p & 31;
    // p >> 5 < 2^26 for any int G, so the chunk term fits its 28 bits
    const uint64_t key = p < B ? ((uint64_t)(s & 7) << 32) | ((uint64_t)(3 - (s >> 3)) << 28) |
                                     (uint64_t)(0x0FFFFFFF - (p >> 5))
                               : (8ull << 32) | (uint64_t)p;
    if (key < best) {
      best = key;
      z = v;
    }
  }
  return z;
}

__device__ __forceinline__ float clamp_q(float v) {
  v = (v < 0.0f) ? 0.0f : v;
  v = (v > 15.0f) ? 15.0f : v;
  return v;
}

template <class IN, int CPT>
__device__ __forceinline__ void load_row(const typename IN::T* p, typename IN::T b[CPT]) {
  if constexpr (CPT == 4) {
    IN::load4(p, b);
  } else {
#pragma unroll
    for (int c = 0; c < CPT; ++c) b[c] = p[c];
  }
}

// One thread quantises CPT adjacent columns of one group (G % 8 == 0).
template <class IN, int CPT>
__global__ __launch_bounds__(256) void quantize_kernel(const typename IN::T* __restrict__ W,
                                                       uint32_t* __restrict__ QW,
                                                       uint16_t* __restrict__ SC,
                                                       uint16_t* __restrict__ ZR, int K, int N,
                                                       int G, int32_t* __restrict__ flag) {
  typedef typename IN::T T;
  const int n = (blockIdx.y * 256 + threadIdx.x) * CPT;
  const int g = blockIdx.x;
  if (n >= N) return;
  const T* src = W + (size_t)g * G * N + n;
  // CPT divides 32 and n is a multiple of CPT: all CPT columns lie on one side.
  static_assert(32 % CPT == 0, "a thread's columns must not straddle a 32-column block");
  const bool tie_last = n < 32 * (N / 32);

  float mn[CPT], mx[CPT];
  bool bad = false;
  {
    T b[CPT];
    load_row<IN, CPT>(src, b);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      bad |= IN::nonfinite(b[c]);
      mn[c] = mx[c] = IN::val(b[c]);
    }
  }
  for (int r = 1; r < G; ++r) {
    T b[CPT];
    load_row<IN, CPT>(src + (size_t)r * N, b);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      bad |= IN::nonfinite(b[c]);
      const float v = IN::val(b[c]);
      mn[c] = min_step(v, mn[c], tie_last);
      mx[c] = (v >= mx[c]) ? v : mx[c];
    }
  }
  if (bad) *flag = 1;
  if constexpr (CPT == 1) {
    if (N == 1 && G >= 32 && mn[0] == 0.0f) mn[0] = inner_zero_min<IN>(src, G);
  }

  float sc[CPT], zr[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    float s = (mx[c] - mn[c]) / 15.0f;
    s = (s > 0.0f) ? s : 1.0f;
    sc[c] = s;
    zr[c] = clamp_q(__builtin_rintf(-mn[c] / s));
  }

  for (int r8 = 0; r8 < G / 8; ++r8) {
    uint32_t word[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) word[c] = 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      T b[CPT];
      load_row<IN, CPT>(src + (size_t)(r8 * 8 + j) * N, b);
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const float q = clamp_q(__builtin_rintf(IN::val(b[c]) / sc[c]) + zr[c]);
        word[c] |= ((uint32_t)(int)q & 0xFu) << (4 * j);
      }
    }
    uint32_t* dst = QW + (size_t)(g * (G / 8) + r8) * N + n;
    if constexpr (CPT == 4) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(word[0], word[1], word[2], word[3]);
    } else {
#pragma unroll
      for (int c = 0; c < CPT; ++c) dst[c] = word[c];
    }
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    SC[(size_t)g * N + n + c] = as_u16((f16)sc[c]);
    ZR[(size_t)g * N + n + c] = as_u16((f16)zr[c]);
  }
}

// Four adjacent columns' weights of one row: 8 (fp16) or 16 (fp32) bytes.
template <class IN>
struct Row4;
template <>
struct Row4<InF16> {
  uint2 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ uint16_t bits(int c) const {
    return (uint16_t)(((c < 2 ? v.x : v.y) >> (16 * (c & 1))) & 0xFFFFu);
  }
  __device__ __forceinline__ float val(int c) const { return InF16::val(bits(c)); }
  __device__ __forceinline__ bool nonfinite(int c) const { return InF16::nonfinite(bits(c)); }
};
template <>
struct Row4<InF32> {
  float4 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ float val(int c) const {
    return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
  }
  __device__ __forceinline__ bool nonfinite(int c) const { return InF32::nonfinite(val(c)); }
};

// One workgroup quantises one group (G rows, G % 8 == 0) of 256 columns
// (N % 4 == 0): lane l of each wave owns columns 4l..4l+3, and wave w a
// contiguous quarter of the group's packed rows (octets).  Every lane issues
// all of its rows' loads at once (the group's min / max no longer waits for
// one row after another), the waves' minima and maxima meet in LDS in wave
// (k) order, and the codes come from the rows still in registers (OPW > 0:
// at most OPW octets per wave) or from a second read of the group (OPW = 0,
// long groups; the tile is L2-resident).  The running minimum's tie rule
// (min_step) applied within a wave in k order and across the waves in k order
// gives the same zero as one scan in k order.  Grid: K / G x N / 256
// workgroups (512 at K = N = 4096, G = 128, against 128 for one thread per
// group and 4 columns).
template <class IN, int OPW>
__global__ __launch_bounds__(256) void quantize_tile_kernel(const typename IN::T* __restrict__ W,
                                                            uint32_t* __restrict__ QW,
                                                            uint16_t* __restrict__ SC,
                                                            uint16_t* __restrict__ ZR, int K,
                                                            int N, int G,
                                                            int32_t* __restrict__ flag) {
  __shared__ float smn[4][256], smx[4][256];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.x;
  const int n = blockIdx.y * 256 + 4 * lane;
  const bool nv = n < N;
  const int octs = G / 8;
  const int per = (octs + 3) / 4;
  const int o0 = min(octs, wave * per), o1 = min(octs, o0 + per);
  const bool tie_last = n < 32 * (N / 32);
  const typename IN::T* src = W + (size_t)g * G * N + n;

  float mn[4], mx[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    mn[c] = __builtin_inff();
    mx[c] = -__builtin_inff();
  }
  bool bad = false;
  auto scan = [&](const Row4<IN>& r) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bad |= r.nonfinite(c);
      const float v = r.val(c);
      mn[c] = min_step(v, mn[c], tie_last);
      mx[c] = (v >= mx[c]) ? v : mx[c];
    }
  };
  Row4<IN> keep[OPW > 0 ? OPW : 1][8];
  if constexpr (OPW > 0) {
#pragma unroll
    for (int i = 0; i < OPW; ++i)
      if (nv && o0 + i < o1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) keep[i][j].load(src + (size_t)((o0 + i) * 8 + j) * N);
      }
#pragma unroll
    for (int i = 0; i < OPW; ++i)
      if (nv && o0 + i < o1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) scan(keep[i][j]);
      }
  } else if (nv) {
    for (int o = o0; o < o1; ++o) {
      Row4<IN> r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j].load(src + (size_t)(o * 8 + j) * N);
#pragma unroll
      for (int j = 0; j < 8; ++j) scan(r[j]);
    }
  }
  if (bad) *flag = 1;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    smn[wave][4 * lane + c] = mn[c];
    smx[wave][4 * lane + c] = mx[c];
  }
  __syncthreads();
  float sc[4], zr[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float a = smn[0][4 * lane + c], b = smx[0][4 * lane + c];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float v = smn[w][4 * lane + c], u = smx[w][4 * lane + c];
      a = min_step(v, a, tie_last);
      b = (u >= b) ? u : b;
    }
    float s = (b - a) / 15.0f;
    s = (s > 0.0f) ? s : 1.0f;
    sc[c] = s;
    zr[c] = clamp_q(__builtin_rintf(-a / s));
  }
  if (!nv) return;
  auto codes = [&](const Row4<IN>(&r)[8], int o) {
    uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float q = clamp_q(__builtin_rintf(r[j].val(c) / sc[c]) + zr[c]);
        word[c] |= ((uint32_t)(int)q & 0xFu) << (4 * j);
      }
    *reinterpret_cast<uint4*>(QW + (size_t)(g * octs + o) * N + n) =
        make_uint4(word[0], word[1], word[2], word[3]);
  };
  if constexpr (OPW > 0) {
#pragma unroll
    for (int i = 0; i < OPW; ++i)
      if (o0 + i < o1) codes(keep[i], o0 + i);
  } else {
    for (int o = o0; o < o1; ++o) {
      Row4<IN> r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j].load(src + (size_t)(o * 8 + j) * N);
      codes(r, o);
    }
  }
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      SC[(size_t)g * N + n + c] = as_u16((f16)sc[c]);
      ZR[(size_t)g * N + n + c] = as_u16((f16)zr[c]);
    }
  }
}

// Any G dividing K (G % 8 != 0 lets a packed word straddle groups): one thread
// per packed word; each row's group statistics are recomputed from the group's
// G values, and the thread that owns a group's first row writes its scale/zero.
struct GroupQ {
  float scale, zero;
  bool bad;
};

template <class IN>
__device__ GroupQ group_stats(const typename IN::T* __restrict__ W, int g, int G, int N, int n) {
  const typename IN::T* src = W + (size_t)g * G * N + n;
  typename IN::T b = src[0];
  bool bad = IN::nonfinite(b);
  float mn = IN::val(b), mx = mn;
  const bool tie_last = n < 32 * (N / 32);
  for (int r = 1; r < G; ++r) {
    b = src[(size_t)r * N];
    bad |= IN::nonfinite(b);
    const float v = IN::val(b);
    mn = min_step(v, mn, tie_last);
    mx = (v >= mx) ? v : mx;
  }
  if (N == 1 && G >= 32 && mn == 0.0f) mn = inner_zero_min<IN>(src, G);
  float s = (mx - mn) / 15.0f;
  s = (s > 0.0f) ? s : 1.0f;
  return GroupQ{s, clamp_q(__builtin_rintf(-mn / s)), bad};
}

template <class IN>
__global__ __launch_bounds__(256) void quantize_general_kernel(
    const typename IN::T* __restrict__ W, uint32_t* __restrict__ QW, uint16_t* __restrict__ SC,
    uint16_t* __restrict__ ZR, int K, int N, int G, int32_t* __restrict__ flag) {
  const int n = blockIdx.y * 256 + threadIdx.x;
  const int i = blockIdx.x;
  if (n >= N) return;
  uint32_t word = 0u;
  int gcur = -1;
  GroupQ gq{1.0f, 0.0f, false};
  bool bad = false;
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * i + j;
    const int g = k / G;
    if (g != gcur) {
      gcur = g;
      gq = group_stats<IN>(W, g, G, N, n);
      bad |= gq.bad;
      if (k == g * G) {
        SC[(size_t)g * N + n] = as_u16((f16)gq.scale);
        ZR[(size_t)g * N + n] = as_u16((f16)gq.zero);
      }
    }
    const float q = clamp_q(__builtin_rintf(IN::val(W[(size_t)k * N + n]) / gq.scale) + gq.zero);
    word |= ((uint32_t)(int)q & 0xFu) << (4 * j);
  }
  if (bad) *flag = 1;
  QW[(size_t)i * N + n] = word;
}

// pack_int4: int32 codes [K, N] -> int32 [K/8, N]; flags values outside [0, 15].
__global__ __launch_bounds__(256) void pack_kernel(const int32_t* __restrict__ Q,
                                                   uint32_t* __restrict__ QW, int K, int N,
                                                   int32_t* __restrict__ flag) {
  const int n = blockIdx.y * 256 + threadIdx.x;
  const int i = blockIdx.x;
  if (n >= N) return;
  uint32_t word = 0u;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t v = Q[(size_t)(8 * i + j) * N + n];
    bad |= (v < 0) | (v > 15);
    word |= ((uint32_t)v & 0xFu) << (4 * j);
  }
  if (bad) *flag = 1;
  QW[(size_t)i * N + n] = word;
}

// unpack_int4: int32 [K/8, N] -> int32 codes [K, N].
__global__ __launch_bounds__(256) void unpack_kernel(const uint32_t* __restrict__ QW,
                                                     int32_t* __restrict__ Q, int K, int N) {
  const int n = blockIdx.y * 256 + threadIdx.x;
  const int i = blockIdx.x;
  if (n >= N) return;
  const uint32_t w = QW[(size_t)i * N + n];
#pragma unroll
  for (int j = 0; j < 8; ++j) Q[(size_t)(8 * i + j) * N + n] = (int32_t)((w >> (4 * j)) & 0xFu);
}

// dequantize_weight: fp16 (fp16(q) - z) * s for any fp16 zero-point.
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ QW,
                                                      const f16* __restrict__ SC,
                                                      const f16* __restrict__ ZR,
                                                      f16* __restrict__ Wd, int K, int N, int G) {
  const int n = blockIdx.y * 256 + threadIdx.x;
  const int i = blockIdx.x;
  if (n >= N) return;
  const uint32_t w = QW[(size_t)i * N + n];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int g = (8 * i + j) / G;
    const f16 s = SC[(size_t)g * N + n];
    const f16 z = ZR[(size_t)g * N + n];
    const f16 q = (f16)(float)((w >> (4 * j)) & 0xFu);
    Wd[(size_t)(8 * i + j) * N + n] = (q - z) * s;
  }
}

// Zero-points outside the integer-zero kernels' domain (w4a16_device.h): any
// zero that is not an integer in [-1024, 1024] (NaN and infinities included)
// sets *flag.  Grid-stride over the n halves; every offending lane stores 1.
__global__ __launch_bounds__(256) void zeros_check_kernel(const f16* __restrict__ Z, int64_t n,
                                                          int32_t* __restrict__ flag) {
  bool bad = false;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float z = (float)Z[i];
    bad |= !(z == __builtin_rintf(z) && __builtin_fabsf(z) <= 1024.0f);
  }
  if (bad) *flag = 1;
}

template <class IN>
hipError_t quantize_launch(const void* W, int32_t* qw, void* sc, void* zr, int K, int N, int G,
                           int32_t* flag, hipStream_t st) {
  typedef typename IN::T T;
  const T* w = static_cast<const T*>(W);
  uint32_t* q = reinterpret_cast<uint32_t*>(qw);
  uint16_t* s = static_cast<uint16_t*>(sc);
  uint16_t* z = static_cast<uint16_t*>(zr);
  if (G % 8 != 0) {
    dim3 grid(K / 8, (N + 255) / 256);
    hipLaunchKernelGGL(quantize_general_kernel<IN>, grid, dim3(256), 0, st, w, q, s, z, K, N, G,
                       flag);
    return hipGetLastError();
  }
  const uintptr_t wa = 4 * sizeof(T);
  const bool vec = (N % 4 == 0) && ((reinterpret_cast<uintptr_t>(W) & (wa - 1)) == 0) &&
                   ((reinterpret_cast<uintptr_t>(qw) & 15) == 0);
  if (vec) {
    // octets per wave: kept in registers up to 8 (fp16) / 4 (fp32), beyond
    // that read twice
    const int per = (G / 8 + 3) / 4;
    constexpr int kMaxKeep = sizeof(T) == 2 ? 8 : 4;
    auto k = per <= 1 ? quantize_tile_kernel<IN, 1>
             : per <= 2 ? quantize_tile_kernel<IN, 2>
             : per <= 4 ? quantize_tile_kernel<IN, 4>
             : per <= kMaxKeep ? quantize_tile_kernel<IN, kMaxKeep>
                              : quantize_tile_kernel<IN, 0>;
    dim3 grid(K / G, (N + 255) / 256);
    hipLaunchKernelGGL(k, grid, dim3(256), 0, st, w, q, s, z, K, N, G, flag);
  } else {
    dim3 grid(K / G, (N + 255) / 256);
    hipLaunchKernelGGL((quantize_kernel<IN, 1>), grid, dim3(256), 0, st, w, q, s, z, K, N, G,
                       flag);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize_pack(const void* W, bool w_is_f32, int32_t* qw, void* sc, void* zr,
                                int K, int N, int G, int32_t* flag, hipStream_t st) {
  return w_is_f32 ? quantize_launch<InF32>(W, qw, sc, zr, K, N, G, flag, st)
                  : quantize_launch<InF16>(W, qw, sc, zr, K, N, G, flag, st);
}

hipError_t launch_pack(const int32_t* q, int32_t* qw, int K, int N, int32_t* flag,
                       hipStream_t st) {
  dim3 grid(K / 8, (N + 255) / 256);
  hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, st, q, reinterpret_cast<uint32_t*>(qw), K,
                     N, flag);
  return hipGetLastError();
}

hipError_t launch_unpack(const int32_t* qw, int32_t* q, int K, int N, hipStream_t st) {
  dim3 grid(K / 8, (N + 255) / 256);
  hipLaunchKernelGGL(unpack_kernel, grid, dim3(256), 0, st,
                     reinterpret_cast<const uint32_t*>(qw), q, K, N);
  return hipGetLastError();
}

hipError_t launch_zeros_check(const void* zr, int64_t n, int32_t* flag, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(zeros_check_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256),
                     0, st, static_cast<const f16*>(zr), n, flag);
  return hipGetLastError();
}

hipError_t launch_dequant(const int32_t* qw, const void* sc, const void* zr, void* w, int K,
                          int N, int G, hipStream_t st) {
  dim3 grid(K / 8, (N + 255) / 256);
  hipLaunchKernelGGL(dequant_kernel, grid, dim3(256), 0, st,
                     reinterpret_cast<const uint32_t*>(qw), static_cast<const f16*>(sc),
                     static_cast<const f16*>(zr), static_cast<f16*>(w), K, N, G);
  return hipGetLastError();
}

}  // namespace w4a16
