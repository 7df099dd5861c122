// Loads-only floor probe for the decode GEMV (a measurement tool, built into
// its own library, libw4a16_floor_probe.so; nothing in libw4a16.so uses it).
//
// It reads packed weights exactly the way the GEMV's workgroups do and does
// nothing with them but an xor, so its time per call is what the access shape
// alone costs: the floor under the GEMV for that shape.
//
//   * rows: a workgroup owns a column block of CWB bytes (16 lanes x 4 bytes
//     = 64 B for a 16-column GEMV block) over all KP packed rows; CWB / 16
//     lanes cover a row segment with one 16-byte non-temporal load each; the
//     rows are dealt to the row-lanes in sweeps (slot j of row-lane rl is row
//     j * RL + rl), BR rows per lane per batch, the next batch issued before
//     the current one is consumed; XCD-aware block order as in the GEMV;
//   * linear: workgroup b reads the contiguous bytes [b * chunk, (b + 1) *
//     chunk), 16 bytes per lane per load, BR loads per lane in flight.
// Each thread writes one word (the xor of what it read) so that no load is
// dead; `out` holds gridDim.x * blockDim.x words.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// past the buffer's range a raw buffer load returns zero and reads nothing
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2 /* nt */);
}

template <int CWB, int WAVES, int BR>
__global__ __launch_bounds__(64 * WAVES) void rows_kernel(const uint8_t* __restrict__ w, int KP,
                                                          int row_bytes, int nb,
                                                          uint32_t* __restrict__ out) {
  constexpr int LPR = CWB / 16;            // lanes per row segment
  constexpr int RW = 64 / LPR;             // row-lanes per wave
  constexpr int RL = WAVES * RW;           // row-lanes per workgroup
  int lin = (int)blockIdx.x;
  if ((nb & 7) == 0) lin = (lin & 7) * (nb >> 3) + (lin >> 3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rl = wave * RW + lane / LPR;
  const uint32_t col = (uint32_t)lin * CWB + (uint32_t)(lane % LPR) * 16u;
  const __amdgpu_buffer_rsrc_t r = rsrc(w, (uint32_t)KP * (uint32_t)row_bytes);
  const int nbat = (KP + BR * RL - 1) / (BR * RL);
  u32x4 a[BR], b[BR];
  u32x4 acc = {0u, 0u, 0u, 0u};
  auto load = [&](int bi, u32x4(&d)[BR]) {
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      const int row = (bi * BR + i) * RL + rl;
      d[i] = load16(r, row < KP ? (uint32_t)row * (uint32_t)row_bytes + col : kOob);
    }
  };
  load(0, a);
  for (int bi = 0; bi < nbat; bi += 2) {
    load(bi + 1, b);
#pragma unroll
    for (int i = 0; i < BR; ++i) acc ^= a[i];
    if (bi + 1 >= nbat) break;
    load(bi + 2, a);
#pragma unroll
    for (int i = 0; i < BR; ++i) acc ^= b[i];
  }
  out[(size_t)blockIdx.x * blockDim.x + tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

template <int WAVES, int BR>
__global__ __launch_bounds__(64 * WAVES) void linear_kernel(const uint8_t* __restrict__ w,
                                                            uint32_t bytes, uint32_t chunk,
                                                            uint32_t* __restrict__ out) {
  constexpr uint32_t kStep = 64u * WAVES * 16u;   // bytes per wave-set load
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t r = rsrc(w, bytes);
  const uint32_t base = blockIdx.x * chunk;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint32_t o = 0; o < chunk; o += kStep * BR) {
    u32x4 d[BR];
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      const uint32_t off = o + (uint32_t)i * kStep + (uint32_t)tid * 16u;
      d[i] = load16(r, off < chunk ? base + off : kOob);
    }
#pragma unroll
    for (int i = 0; i < BR; ++i) acc ^= d[i];
  }
  out[(size_t)blockIdx.x * blockDim.x + tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// tiles: workgroup -> (column block cb of CWB bytes, k-range ks of S equal
// ranges), placed like the GEMV's blocks (consecutive (cb, ks) on one XCD); the
// loads are rows_kernel's over the range's KP / S rows.  Each lane's xor, read
// as four floats (one per column of its 16 bytes), is summed over the
// workgroup's row-lanes in LDS into one float per column: the workgroup's
// partial.  MODE 0: the partial is stored to out[(cb * S + ks) * CW + c] (the
// access shape alone, no cross-workgroup step).  MODE 1: the k-ranges are summed
// inside the kernel without a fence: device-coherent partial stores (sc1), a
// wait for their completion, one device-scope atomic add on the column block's
// counter; the workgroup that arrives last loads the S partials with
// device-coherent loads, sums them in range order, stores the block's result to
// out[cb * CW + c] and resets the counter to zero for the next call (the
// counters start at zero).  MODE 2: as MODE 1 with plain stores and loads: the
// cost of the same chain through the L2 alone, which is only coherent when the
// S workgroups of a block share an XCD (timing only; its sums are not checked).
template <int CWB, int WAVES, int BR, int MODE>
__global__ __launch_bounds__(64 * WAVES) void tiles_kernel(const uint8_t* __restrict__ w, int KP,
                                                           int row_bytes, int S, int nb,
                                                           float* __restrict__ part,
                                                           uint32_t* __restrict__ cnt,
                                                           float* __restrict__ out) {
  constexpr int LPR = CWB / 16;            // lanes per row segment
  constexpr int RW = 64 / LPR;             // row-lanes per wave
  constexpr int RL = WAVES * RW;           // row-lanes per workgroup
  constexpr int CW = CWB / 4;              // columns per block
  __shared__ float red[RL][CW];
  __shared__ uint32_t last;
  int lin = (int)blockIdx.x;
  if ((nb & 7) == 0) lin = (lin & 7) * (nb >> 3) + (lin >> 3);
  const int cb = lin / S, ks = lin - cb * S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rl = wave * RW + lane / LPR;
  const uint32_t col = (uint32_t)cb * CWB + (uint32_t)(lane % LPR) * 16u;
  const int rows = KP / S, rb = ks * rows;
  const __amdgpu_buffer_rsrc_t r = rsrc(w, (uint32_t)KP * (uint32_t)row_bytes);
  const int nbat = (rows + BR * RL - 1) / (BR * RL);
  u32x4 a[BR], b[BR];
  u32x4 acc = {0u, 0u, 0u, 0u};
  auto load = [&](int bi, u32x4(&d)[BR]) {
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      const int row = (bi * BR + i) * RL + rl;
      d[i] = load16(r, row < rows ? (uint32_t)(rb + row) * (uint32_t)row_bytes + col : kOob);
    }
  };
  load(0, a);
  for (int bi = 0; bi < nbat; bi += 2) {
    load(bi + 1, b);
#pragma unroll
    for (int i = 0; i < BR; ++i) acc ^= a[i];
    if (bi + 1 >= nbat) break;
    load(bi + 2, a);
#pragma unroll
    for (int i = 0; i < BR; ++i) acc ^= b[i];
  }
  // finite floats whatever the bits: keep the mantissa, fix the exponent
  const int c0 = 4 * (lane % LPR);
  red[rl][c0 + 0] = __uint_as_float((acc.x & 0x007FFFFFu) | 0x3F800000u);
  red[rl][c0 + 1] = __uint_as_float((acc.y & 0x007FFFFFu) | 0x3F800000u);
  red[rl][c0 + 2] = __uint_as_float((acc.z & 0x007FFFFFu) | 0x3F800000u);
  red[rl][c0 + 3] = __uint_as_float((acc.w & 0x007FFFFFu) | 0x3F800000u);
  __syncthreads();
  float v = 0.0f;
  if (tid < CW)
    for (int i = 0; i < RL; ++i) v += red[i][tid];
  if constexpr (MODE == 0) {
    if (tid < CW) out[(size_t)lin * CW + tid] = v;
    return;
  } else {
    if (tid < CW) {
      if constexpr (MODE == 1)
        __hip_atomic_store(&part[(size_t)lin * CW + tid], v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      else
        part[(size_t)lin * CW + tid] = v;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(&cnt[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(S - 1);
    __syncthreads();
    if (last) {
      if (tid < CW) {
        float s = 0.0f;
        for (int k = 0; k < S; ++k) {
          const float* p = &part[((size_t)cb * S + k) * CW + tid];
          if constexpr (MODE == 1)
            s += __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            s += *p;
        }
        out[(size_t)cb * CW + tid] = s;
      }
      if (tid == 0) __hip_atomic_store(&cnt[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int CWB, int WAVES, int BR>
int launch_rows(const void* w, int KP, int row_bytes, uint32_t* out, hipStream_t st) {
  hipLaunchKernelGGL((rows_kernel<CWB, WAVES, BR>), dim3(row_bytes / CWB), dim3(64 * WAVES), 0, st,
                     static_cast<const uint8_t*>(w), KP, row_bytes, row_bytes / CWB, out);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

// Words `out` must hold for a rows / linear launch.
int64_t w4a16_probe_rows_out_words(int row_bytes, int cwb, int waves) {
  return (int64_t)(row_bytes / cwb) * 64 * waves;
}
int64_t w4a16_probe_linear_out_words(int nwg, int waves) { return (int64_t)nwg * 64 * waves; }

// rows: (cwb, waves, br) in {(64, 16, 2), (64, 8, 4), (128, 16, 2), (256, 8, 4),
// (256, 16, 2), (512, 8, 4), (512, 16, 2)}; row_bytes % cwb == 0,
// KP * row_bytes < 2 GiB.
// Returns 0, a HIP error, or -1 for an unsupported shape.
int w4a16_probe_rows(const void* w, int KP, int row_bytes, int cwb, int waves, int br, uint32_t* out,
                     hipStream_t st) {
  if (KP <= 0 || row_bytes <= 0 || cwb <= 0 || row_bytes % cwb != 0 ||
      (int64_t)KP * row_bytes >= ((int64_t)1 << 31))
    return -1;
  if (cwb == 64 && waves == 16 && br == 2) return launch_rows<64, 16, 2>(w, KP, row_bytes, out, st);
  if (cwb == 64 && waves == 8 && br == 4) return launch_rows<64, 8, 4>(w, KP, row_bytes, out, st);
  if (cwb == 128 && waves == 16 && br == 2) return launch_rows<128, 16, 2>(w, KP, row_bytes, out, st);
  if (cwb == 256 && waves == 8 && br == 4) return launch_rows<256, 8, 4>(w, KP, row_bytes, out, st);
  if (cwb == 256 && waves == 16 && br == 2) return launch_rows<256, 16, 2>(w, KP, row_bytes, out, st);
  if (cwb == 512 && waves == 8 && br == 4) return launch_rows<512, 8, 4>(w, KP, row_bytes, out, st);
  if (cwb == 512 && waves == 16 && br == 2) return launch_rows<512, 16, 2>(w, KP, row_bytes, out, st);
  return -1;
}

// tiles: (cwb, waves, br) in {(128, 8, 4), (256, 8, 4), (512, 8, 4)}, mode 0 / 1 / 2;
// row_bytes % cwb == 0, KP % s == 0, KP * row_bytes < 2 GiB.  `part` holds
// (row_bytes / cwb) * s * cwb / 4 floats, `cnt` row_bytes / cwb zeroed words
// (left zeroed by every mode-1/2 call), `out` as many floats as `part`.
int w4a16_probe_tiles(const void* w, int KP, int row_bytes, int cwb, int waves, int br, int s,
                      int mode, float* part, uint32_t* cnt, float* out, hipStream_t st) {
  if (KP <= 0 || row_bytes <= 0 || cwb <= 0 || row_bytes % cwb != 0 || s <= 0 || KP % s != 0 ||
      (int64_t)KP * row_bytes >= ((int64_t)1 << 31) || waves != 8 || br != 4 || mode < 0 ||
      mode > 2)
    return -1;
  const dim3 grid((unsigned)(row_bytes / cwb * s)), block(512);
  const uint8_t* wp = static_cast<const uint8_t*>(w);
#define W4A16_PROBE_TILES(CWB)                                                                   \
  if (cwb == CWB) {                                                                              \
    if (mode == 0)                                                                               \
      hipLaunchKernelGGL((tiles_kernel<CWB, 8, 4, 0>), grid, block, 0, st, wp, KP, row_bytes, s, \
                         (int)grid.x, part, cnt, out);                                           \
    else if (mode == 1)                                                                          \
      hipLaunchKernelGGL((tiles_kernel<CWB, 8, 4, 1>), grid, block, 0, st, wp, KP, row_bytes, s, \
                         (int)grid.x, part, cnt, out);                                           \
    else                                                                                         \
      hipLaunchKernelGGL((tiles_kernel<CWB, 8, 4, 2>), grid, block, 0, st, wp, KP, row_bytes, s, \
                         (int)grid.x, part, cnt, out);                                           \
    return (int)hipGetLastError();                                                               \
  }
  W4A16_PROBE_TILES(128)
  W4A16_PROBE_TILES(256)
  W4A16_PROBE_TILES(512)
#undef W4A16_PROBE_TILES
  return -1;
}

// linear: waves 8 with br 4, or waves 4 with br 8; bytes % (16 * nwg) == 0,
// bytes < 2 GiB.
int w4a16_probe_linear(const void* w, uint32_t bytes, int nwg, int waves, int br, uint32_t* out,
                       hipStream_t st) {
  if (nwg <= 0 || bytes % (16u * (uint32_t)nwg) != 0 || bytes >= (1u << 31)) return -1;
  const uint32_t chunk = bytes / (uint32_t)nwg;
  if (waves == 8 && br == 4)
    hipLaunchKernelGGL((linear_kernel<8, 4>), dim3(nwg), dim3(512), 0, st,
                       static_cast<const uint8_t*>(w), bytes, chunk, out);
  else if (waves == 4 && br == 8)
    hipLaunchKernelGGL((linear_kernel<4, 8>), dim3(nwg), dim3(256), 0, st,
                       static_cast<const uint8_t*>(w), bytes, chunk, out);
  else
    return -1;
  return (int)hipGetLastError();
}

}  // extern "C"
