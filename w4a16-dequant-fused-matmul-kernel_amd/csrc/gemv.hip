// Decode GEMV for small M (M <= 8): Y = X @ dequant(qweight) streamed from HBM.
//
// Replaces the decode regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128 at M = 1..16, BLOCK_M >= 16).
//
// Layout of the work:
//   * a workgroup is 4 waves; all 64 lanes of a wave sit on one packed row and
//     4 consecutive columns each (one global_load_dwordx4 = 256 columns = 1 KiB);
//   * the 4 waves split the workgroup's packed rows into contiguous sub-blocks,
//     so each wave's group index changes every G/8 rows (uniform branch);
//   * activations are wave-uniform per row and are read through the scalar
//     cache into SGPRs (8 halves per row and activation row);
//   * dequant is the packed-fp16 magic-number form (w4a16_device.h) and the dot
//     product is v_dot2_f32_f16 with fp32 accumulation; no MFMA is used;
//   * the 4 waves' partial sums meet in LDS in a fixed order; with a k-split
//     (grid.y > 1) each workgroup writes fp32 partials and the last workgroup of
//     a column block (atomic counter) sums the splits in split order, so the
//     result does not depend on scheduling.  The last workgroup resets its
//     counter, leaving the workspace ready for the next call.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 8;

template <int MT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(
    const f16* __restrict__ X, const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ bias, f16* __restrict__ Y,
    float* __restrict__ part, uint32_t* __restrict__ cnt, int N, int K, int G, int rows_per_wg,
    int S) {
  __shared__ float red[kWaves][MT][kGemvCols];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cb = blockIdx.x;
  const int sk = blockIdx.y;
  const int n = cb * kGemvCols + lane * 4;
  const bool nv = n < N;
  const int KP = K >> 3;
  const int rb = sk * rows_per_wg;
  const int re = min(KP, rb + rows_per_wg);
  const int per_wave = (re - rb + kWaves - 1) / kWaves;
  const int wb = min(re, rb + wave * per_wave);
  const int we = min(re, wb + per_wave);

  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  int gcur = -1;
  ColQ cq[4];
  for (int r0 = wb; r0 < we; r0 += kUnroll) {
    uint4 wv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = r0 + u;
      wv[u] = (nv && r < we) ? *reinterpret_cast<const uint4*>(QW + (size_t)r * N + n)
                             : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = r0 + u;
      if (r >= we) break;
      const int g = (r * 8) / G;
      if (g != gcur) {
        gcur = g;
        uint2 sv = make_uint2(0x3C003C00u, 0x3C003C00u);
        uint2 zv = make_uint2(0u, 0u);
        if (nv) {
          sv = *reinterpret_cast<const uint2*>(SC + (size_t)g * N + n);
          zv = *reinterpret_cast<const uint2*>(ZR + (size_t)g * N + n);
        }
        cq[0] = make_colq(sv.x & 0xFFFFu, zv.x & 0xFFFFu);
        cq[1] = make_colq(sv.x >> 16, zv.x >> 16);
        cq[2] = make_colq(sv.y & 0xFFFFu, zv.y & 0xFFFFu);
        cq[3] = make_colq(sv.y >> 16, zv.y >> 16);
      }
      f16x2 d[4][4];
      dq_word(wv[u].x, cq[0], d[0]);
      dq_word(wv[u].y, cq[1], d[1]);
      dq_word(wv[u].z, cq[2], d[2]);
      dq_word(wv[u].w, cq[3], d[3]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const uint4 xr = *reinterpret_cast<const uint4*>(X + (size_t)m * K + (size_t)r * 8);
        const uint4 xp = perm_pairs(xr);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float a = acc[m][c];
          a = __builtin_amdgcn_fdot2(d[c][0], as_h2(xp.x), a, false);
          a = __builtin_amdgcn_fdot2(d[c][1], as_h2(xp.y), a, false);
          a = __builtin_amdgcn_fdot2(d[c][2], as_h2(xp.z), a, false);
          a = __builtin_amdgcn_fdot2(d[c][3], as_h2(xp.w), a, false);
          acc[m][c] = a;
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m)
    *reinterpret_cast<float4*>(&red[wave][m][lane * 4]) =
        make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
  __syncthreads();

  const int t = threadIdx.x;
  const int col = cb * kGemvCols + t;
  const bool cv = col < N;
  float v[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float s = red[0][m][t];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[w][m][t];
    v[m] = s;
  }

  if (S == 1) {
    if (cv) {
      const f16 b = bias ? bias[col] : (f16)0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        f16 y = f32_to_f16(v[m]);
        if (bias) y = y + b;
        Y[(size_t)m * N + col] = y;
      }
    }
    return;
  }

  if (cv) {
#pragma unroll
    for (int m = 0; m < MT; ++m) part[((size_t)sk * MT + m) * N + col] = v[m];
  }
  __threadfence();
  __syncthreads();
  if (t == 0) s_last = (atomicAdd(&cnt[cb], 1u) == (uint32_t)(S - 1)) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (cv) {
    const f16 b = bias ? bias[col] : (f16)0.0f;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float s = 0.0f;
      for (int q = 0; q < S; ++q) s += part[((size_t)q * MT + m) * N + col];
      f16 y = f32_to_f16(s);
      if (bias) y = y + b;
      Y[(size_t)m * N + col] = y;
    }
  }
  if (t == 0) cnt[cb] = 0u;
}

template <int MT>
hipError_t launch_mt(const GemmArgs& a, int split, void* ws, hipStream_t st) {
  const int nblk = (a.N + kGemvCols - 1) / kGemvCols;
  const int rows = gemv_rows_per_split(a.K, split);
  const int S = split;
  uint32_t* cnt = nullptr;
  float* part = nullptr;
  if (S > 1) {
    cnt = static_cast<uint32_t*>(ws);
    const size_t cnt_bytes = ((size_t)nblk * 4 + 255) / 256 * 256;
    part = reinterpret_cast<float*>(static_cast<char*>(ws) + cnt_bytes);
  }
  dim3 grid(nblk, S);
  hipLaunchKernelGGL(gemv_kernel<MT>, grid, dim3(kThreads), 0, st,
                     static_cast<const f16*>(a.x), reinterpret_cast<const uint32_t*>(a.qw),
                     static_cast<const uint16_t*>(a.sc), static_cast<const uint16_t*>(a.zr),
                     static_cast<const f16*>(a.bias), static_cast<f16*>(a.y), part, cnt, a.N, a.K,
                     a.G, rows, S);
  return hipGetLastError();
}

}  // namespace

int gemv_rows_per_split(int K, int split) {
  const int KP = K / 8;
  return (KP + split - 1) / split;
}

size_t gemv_workspace_bytes(int M, int N, int K, int split) {
  (void)K;
  if (split <= 1) return 0;
  const size_t nblk = (size_t)(N + kGemvCols - 1) / kGemvCols;
  const size_t cnt_bytes = (nblk * 4 + 255) / 256 * 256;
  return cnt_bytes + (size_t)split * (size_t)M * (size_t)N * sizeof(float);
}

hipError_t launch_gemv(const GemmArgs& a, int split, void* ws, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_mt<1>(a, split, ws, st);
    case 2: return launch_mt<2>(a, split, ws, st);
    case 3: return launch_mt<3>(a, split, ws, st);
    case 4: return launch_mt<4>(a, split, ws, st);
    case 5: return launch_mt<5>(a, split, ws, st);
    case 6: return launch_mt<6>(a, split, ws, st);
    case 7: return launch_mt<7>(a, split, ws, st);
    case 8: return launch_mt<8>(a, split, ws, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
