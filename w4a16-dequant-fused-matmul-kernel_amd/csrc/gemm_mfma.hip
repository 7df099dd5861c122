// Prefill W4A16 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x16_f16).
//
// Replaces the prefill regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128: fp16 dequant of the weight
// tile, tl.dot with fp32 accumulation, fp16 store).
//
// Design:
//   * each wave owns (32*WMT) rows x 128 columns of Y; a workgroup is
//     WAVES_M x WAVES_N waves, all sharing one activation tile in LDS;
//   * weights never go through LDS: the B operand of v_mfma_f32_32x32x16_f16 in
//     lane l is 8 consecutive k of column l%32 -- exactly one packed int32 word.
//     Each lane loads one dwordx4 (4 consecutive columns) per packed row and
//     dequantises it in registers (packed fp16, w4a16_device.h), feeding four
//     MFMAs that cover columns {4j + c}; a wave's 4 MFMAs cover 128 columns;
//   * dequant yields k in pair order (0,4,1,5,2,6,3,7); the activation octets are
//     permuted the same way when they are written to LDS, so A and B agree on k;
//   * K advances 64 per step, LDS double-buffered with one barrier per step,
//     next step's A/B/scale loads issued before the current step's MFMAs;
//   * LDS rows are padded to 144 bytes so the ds_read_b128 of 16 rows x 16 B
//     hits 64 distinct banks;
//   * epilogue: lane l holds 4 consecutive columns per output row, rounded to
//     fp16 (RNE) and stored as one 8-byte write; optional fp16 bias add
//     reproduces W4A16Linear's separate `y + bias` (linear.py:90-91).
// Requirements (checked by the caller): N % 4 == 0, G % 32 == 0, K % G == 0,
// 16-byte aligned x/qweight, 8-byte aligned scales/zeros/y/bias.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kBK = 64;
constexpr int kLdsRow = 9;  // uint4 per LDS row: 8 octets + 1 pad

template <int WMT, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void mfma_kernel(
    const f16* __restrict__ X, const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ bias, f16* __restrict__ Y, int M,
    int N, int K, int G) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int BM = 32 * WMT * WAVES_M;
  constexpr int BN = 128 * WAVES_N;
  constexpr int A_PER_T = BM * 8 / NT;
  static_assert((BM * 8) % NT == 0, "A tile must split evenly over threads");
  __shared__ uint4 As[2][BM * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;

  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int ncol = n0 + wn * 128 + 4 * l32;
  const bool nv = ncol < N;
  const int KP = K >> 3;
  const int KT = (K + kBK - 1) / kBK;
  const int NG = K / G;

  f32x16 acc[WMT][4];
#pragma unroll
  for (int i = 0; i < WMT; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = f32x16{};

  uint4 ra[A_PER_T];
  uint4 rb[4], nb[4];
  uint2 rs[2], rz[2], ns[2], nz[2];

  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int o = tid + i * NT;
      const int row = o >> 3, oct = o & 7;
      const int gm = m0 + row;
      const int k = kt * kBK + oct * 8;
      ra[i] = (gm < M && k < K) ? *reinterpret_cast<const uint4*>(X + (size_t)gm * K + k)
                                : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int o = tid + i * NT;
      const int row = o >> 3, oct = o & 7;
      As[buf][row * kLdsRow + oct] = perm_pairs(ra[i]);
    }
  };
  auto load_b = [&](int kt, uint4* dst) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int pr = kt * 8 + 2 * s + lhi;
      dst[s] = (nv && pr < KP) ? *reinterpret_cast<const uint4*>(QW + (size_t)pr * N + ncol)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto load_s = [&](int kt, uint2* sd, uint2* zd) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = min((kt * kBK + 32 * h) / G, NG - 1);
      if (nv) {
        sd[h] = *reinterpret_cast<const uint2*>(SC + (size_t)g * N + ncol);
        zd[h] = *reinterpret_cast<const uint2*>(ZR + (size_t)g * N + ncol);
      } else {
        sd[h] = make_uint2(0x3C003C00u, 0x3C003C00u);
        zd[h] = make_uint2(0u, 0u);
      }
    }
  };

  load_a(0);
  load_b(0, rb);
  load_s(0, rs, rz);
  store_a(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = (kt + 1) < KT;
    if (more) {
      load_a(kt + 1);
      load_b(kt + 1, nb);
      load_s(kt + 1, ns, nz);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      ColQ cq[4];
      cq[0] = make_colq(rs[h].x & 0xFFFFu, rz[h].x & 0xFFFFu);
      cq[1] = make_colq(rs[h].x >> 16, rz[h].x >> 16);
      cq[2] = make_colq(rs[h].y & 0xFFFFu, rz[h].y & 0xFFFFu);
      cq[3] = make_colq(rs[h].y >> 16, rz[h].y >> 16);
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const int s = 2 * h + ss;
        const uint32_t words[4] = {rb[s].x, rb[s].y, rb[s].z, rb[s].w};
        f16x8 bf[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          f16x2 d[4];
          dq_word(words[c], cq[c], d);
          bf[c] = f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
        }
#pragma unroll
        for (int mt = 0; mt < WMT; ++mt) {
          const int row = wm * (32 * WMT) + mt * 32 + l32;
          const f16x8 af = __builtin_bit_cast(f16x8, As[cur][row * kLdsRow + 2 * s + lhi]);
#pragma unroll
          for (int c = 0; c < 4; ++c)
            acc[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[c], acc[mt][c], 0, 0, 0);
        }
      }
    }
    if (more) {
      store_a(cur ^ 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) rb[s] = nb[s];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        rs[h] = ns[h];
        rz[h] = nz[h];
      }
    }
    __syncthreads();
  }

  if (!nv) return;
  f16 bv[4] = {(f16)0.0f, (f16)0.0f, (f16)0.0f, (f16)0.0f};
  if (bias) {
    const uint2 b2 = *reinterpret_cast<const uint2*>(bias + ncol);
    bv[0] = as_h(b2.x & 0xFFFFu);
    bv[1] = as_h(b2.x >> 16);
    bv[2] = as_h(b2.y & 0xFFFFu);
    bv[3] = as_h(b2.y >> 16);
  }
#pragma unroll
  for (int mt = 0; mt < WMT; ++mt) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int row = m0 + wm * (32 * WMT) + mt * 32 + 8 * (a >> 2) + 4 * lhi + (a & 3);
      if (row < M) {
        f16x4 o;
        o.x = f32_to_f16(acc[mt][0][a]);
        o.y = f32_to_f16(acc[mt][1][a]);
        o.z = f32_to_f16(acc[mt][2][a]);
        o.w = f32_to_f16(acc[mt][3][a]);
        if (bias) {
          o.x = o.x + bv[0];
          o.y = o.y + bv[1];
          o.z = o.z + bv[2];
          o.w = o.w + bv[3];
        }
        *reinterpret_cast<f16x4*>(Y + (size_t)row * N + ncol) = o;
      }
    }
  }
}

template <int WMT, int WAVES_M, int WAVES_N>
hipError_t launch_cfg(const GemmArgs& a, hipStream_t st) {
  constexpr int BM = 32 * WMT * WAVES_M;
  constexpr int BN = 128 * WAVES_N;
  dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  hipLaunchKernelGGL((mfma_kernel<WMT, WAVES_M, WAVES_N>), grid, dim3(64 * WAVES_M * WAVES_N), 0,
                     st, static_cast<const f16*>(a.x), reinterpret_cast<const uint32_t*>(a.qw),
                     static_cast<const uint16_t*>(a.sc), static_cast<const uint16_t*>(a.zr),
                     static_cast<const f16*>(a.bias), static_cast<f16*>(a.y), a.M, a.N, a.K, a.G);
  return hipGetLastError();
}

}  // namespace

// cfg 0: 128 x 512 (4 waves along N, each 128 x 128)
// cfg 1: 128 x 256 (2 x 2 waves, each 64 x 128)
// cfg 2:  32 x 512 (4 waves along N, each 32 x 128)
MfmaTile mfma_tile(int cfg) {
  switch (cfg) {
    case 0: return {128, 512};
    case 1: return {128, 256};
    default: return {32, 512};
  }
}

hipError_t launch_mfma(const GemmArgs& a, int cfg, hipStream_t st) {
  switch (cfg) {
    case 0: return launch_cfg<4, 1, 4>(a, st);
    case 1: return launch_cfg<2, 2, 2>(a, st);
    case 2: return launch_cfg<1, 1, 4>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
