// Prefill W4A16 GEMM on gfx950 matrix cores, two waves per SIMD
// (v_mfma_f32_16x16x32_f16, fp32 accumulation).
//
// Replaces the large-M regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128: fp16 dequant of the weight
// tile, tl.dot with fp32 accumulation, fp16 store).
//
// Design:
//   * each wave owns 128 rows x 64 columns of Y: 8 x 4 tiles of 16 x 16, 128
//     accumulator registers, so every SIMD runs two waves (from two
//     workgroups) and one wave's dequant and memory waits overlap the other's
//     MFMAs;
//   * the B operand of v_mfma_f32_16x16x32_f16 in lane l is 8 consecutive k
//     (octet l/16) of column l%16 -- one packed int32 word.  Columns are
//     interleaved by 4: n-tile c, MFMA column j is column 4j + c of the wave's
//     64.  So one 16-byte load per lane (4 adjacent columns of one packed row)
//     feeds all four n-tiles, and per 64-k step a wave issues two weight loads
//     and, per quantisation group, one scale and one zero load;
//   * weights are dequantised in registers (magic-number packed fp16,
//     w4a16_device.h) in pair order (0,4,1,5,2,6,3,7); activation octets are
//     permuted the same way on their way into LDS, so A and B agree on k;
//   * activations: the workgroup's 64-k slice of A is double-buffered in LDS
//     (rows padded to 144 bytes: the 16-lane fragment reads hit distinct
//     banks), one barrier per k-step;
//   * global loads run a step ahead with one register stage each for
//     activations and weights (a weight register is reloaded as soon as it has
//     been dequantised); rows past M / columns past N read as zero through the
//     buffer range check;
//   * XCD-aware grouped tile order; epilogue: each lane holds 4 consecutive
//     columns of 4 rows per tile, rounded to fp16 (RNE) and stored 8 bytes at a
//     time, with the optional fp16 bias add of W4A16Linear (linear.py:90-91).
// Requirements (checked by the caller): K % 64 == 0, N % 4 == 0, G % 32 == 0,
// K % G == 0, 16-byte aligned x/qweight, 8-byte aligned scales/zeros/y/bias,
// and x, qweight, scales, zeros each below 2 GiB.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kBK = 64;
constexpr int kLdsRow = 9;    // uint4 per LDS row: 8 octets + 1 pad
constexpr int kGroupM = 4;    // M-tiles per group of the tile order
constexpr int kMT = 8;        // 16-row MFMA tiles per wave (128 rows)
constexpr int kNTiles = 4;    // 16-column MFMA tiles per wave (64 columns)

template <int WAVES_M, int WAVES_N, bool G64, bool AZ>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) __attribute__((amdgpu_waves_per_eu(2, 2)))
void occ2_kernel(const f16* __restrict__ X, const uint32_t* __restrict__ QW,
                 const uint16_t* __restrict__ SC, const uint16_t* __restrict__ ZR,
                 const f16* __restrict__ bias, f16* __restrict__ Y, float* __restrict__ part,
                 int M, int N, int K, int G, int KTS, int ldx, int ldy) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int BM = 16 * kMT * WAVES_M;
  constexpr int BN = 16 * kNTiles * WAVES_N;
  constexpr int A_PER_T = BM * 8 / NT;
  static_assert((BM * 8) % NT == 0, "A tile must split evenly over threads");
  __shared__ uint4 As[2][BM * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int l16 = lane & 15;    // column quad (B) / row (A) within a tile
  const int oct = lane >> 4;    // k-octet within a 32-k sub-step

  // XCD-aware grouped tile order: the hardware deals workgroups to the 8 XCDs
  // round-robin; each XCD takes a contiguous run of an order that walks kGroupM
  // M-tiles x all N-tiles per group, so concurrent tiles share A rows and B
  // columns in that XCD's L2.
  // With split-K (part != nullptr) the grid is tiles x splits: workgroup
  // (tile T, split sp) accumulates k-steps [sp*KTS, (sp+1)*KTS).
  const int ntn = (N + BN - 1) / BN;
  const int ntm = (M + BM - 1) / BM;
  const int total = ntn * ntm;
  const int nb = (int)gridDim.x;
  int B = (int)blockIdx.x;
  if ((nb & 7) == 0) B = (B & 7) * (nb >> 3) + (B >> 3);
  const int sp = B / total;
  const int T = B - sp * total;
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * BM;
  const int n0 = (rem / gsz) * BN;
  const int ncol = n0 + wn * (16 * kNTiles) + 4 * l16;   // this lane's 4 columns
  const bool nv = ncol < N;
  const int KP = K >> 3;
  const int KS0 = sp * KTS;                  // this workgroup's k-steps [KS0, KT)
  const int KT = min(K / kBK, KS0 + KTS);
  const int NG = K / G;
  constexpr int NH = G64 ? 1 : 2;   // groups per 64-k step (G % 64 == 0: one)

  const MagicRegs mg = make_magic();
  // rows of X lie ldx elements apart; rows at or past M fall outside the range
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(M - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);

  uint32_t a_off[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int o = tid + i * NT;
    const int gm = m0 + (o >> 3);
    a_off[i] = gm < M ? ((uint32_t)gm * (uint32_t)ldx + (uint32_t)(o & 7) * 8u) * 2u : kOobOffset;
  }
  const uint32_t b_off = nv ? ((uint32_t)oct * (uint32_t)N + (uint32_t)ncol) * 4u : kOobOffset;
  const uint32_t s_off = nv ? (uint32_t)ncol * 2u : kOobOffset;

  struct StageB {
    uint4 b[2];              // half h: packed row 4h + oct, columns ncol .. ncol+3
    uint2 sc[NH], zr[NH];    // the step's group(s), columns ncol .. ncol+3
  };
  uint4 ra[A_PER_T];

  auto load_a = [&](int kt) {
    const uint32_t ak = uniform((uint32_t)kt * (uint32_t)(kBK * 2));
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) ra[i] = buf_load16(rx, a_off[i], ak);
  };
  auto load_w = [&](int kt, int h, StageB& st) {
    st.b[h] = buf_load16(rw, b_off, uniform(((uint32_t)kt * 8u + 4u * (uint32_t)h) * (uint32_t)N * 4u));
  };
  auto load_scales = [&](int kt, StageB& st) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const uint32_t g = uniform((uint32_t)((kt * kBK + 32 * h) / G) * (uint32_t)N * 2u);
      st.sc[h] = buf_load8(rs, s_off, g);
      st.zr[h] = buf_load8(rz, s_off, g);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int o = tid + i * NT;
      As[buf][(o >> 3) * kLdsRow + (o & 7)] = perm_pairs(ra[i]);
    }
  };

  f32x4 acc[kMT][kNTiles];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int c = 0; c < kNTiles; ++c) acc[i][c] = f32x4{};

  const int arow = wm * (16 * kMT) + l16;
  // One k-step from LDS buffer `buf` and the weight registers `st`; each
  // register is reloaded with step kt+1's data as soon as it has been used, so
  // one weight stage suffices (the second wave on the SIMD covers the latency).
  auto step = [&](StageB& st, int kt, int buf) {
    const bool more = kt + 1 < KT;
    ColQ cq[NH][4];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const ColQ2 p01 = make_colq2<AZ>(st.sc[h].x, st.zr[h].x);
      const ColQ2 p23 = make_colq2<AZ>(st.sc[h].y, st.zr[h].y);
      cq[h][0] = colq_of<0>(p01);
      cq[h][1] = colq_of<1>(p01);
      cq[h][2] = colq_of<0>(p23);
      cq[h][3] = colq_of<1>(p23);
    }
    // the next step's group(s); with one group per step (G % 64 == 0) they are
    // reloaded only when the group changes
    const bool same_group = G64 && ((kt + 1) * kBK) / G == (kt * kBK) / G;
    if (more && !same_group) load_scales(kt + 1, st);
    const uint4* A = &As[buf][arow * kLdsRow + oct];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const ColQ* c4 = cq[G64 ? 0 : h];
      const uint32_t words[4] = {st.b[h].x, st.b[h].y, st.b[h].z, st.b[h].w};
      f16x8 bf[kNTiles];
#pragma unroll
      for (int c = 0; c < kNTiles; ++c) {
        f16x2 d[4];
        dq_word_fast<AZ>(words[c], c4[c], mg, d);
        bf[c] = f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
      }
      if (more) load_w(kt + 1, h, st);
      // m-tiles in two groups of four keep 16 fragment registers live
#pragma unroll
      for (int ig = 0; ig < kMT; ig += 4) {
        f16x8 af[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          af[i] = __builtin_bit_cast(f16x8, A[(ig + i) * 16 * kLdsRow + 4 * h]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int c = 0; c < kNTiles; ++c)
            acc[ig + i][c] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[c], acc[ig + i][c], 0, 0, 0);
      }
      // keep the scheduler from hoisting the next half's work above these
      // MFMAs (register pressure at two waves per SIMD)
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  StageB sb;
  load_a(KS0);
  load_w(KS0, 0, sb);
  load_w(KS0, 1, sb);
  load_scales(KS0, sb);
  store_a(0);
  __syncthreads();
  if (KS0 + 1 < KT) load_a(KS0 + 1);
  for (int kt = KS0; kt < KT; ++kt) {
    const int buf = (kt - KS0) & 1;
    step(sb, kt, buf);
    if (kt + 1 < KT) store_a(buf ^ 1);   // step kt+1's activations
    __syncthreads();
    if (kt + 2 < KT) load_a(kt + 2);
  }

  if (part) {
    // fp32 partial sums of this split, 4 columns per lane (16-byte stores)
    if (!nv) return;
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * (16 * kMT) + 16 * i + 4 * oct + r;
        if (row < M)
          *reinterpret_cast<float4*>(part + ((size_t)sp * M + row) * N + ncol) =
              make_float4(acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]);
      }
    return;
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
  for (int i = 0; i < kMT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * (16 * kMT) + 16 * i + 4 * oct + r;
      if (row < M) {
        f16x4 o;
        o.x = f32_to_f16(acc[i][0][r]);
        o.y = f32_to_f16(acc[i][1][r]);
        o.z = f32_to_f16(acc[i][2][r]);
        o.w = f32_to_f16(acc[i][3][r]);
        if (bias) {
          o.x = o.x + bv[0];
          o.y = o.y + bv[1];
          o.z = o.z + bv[2];
          o.w = o.w + bv[3];
        }
        *reinterpret_cast<f16x4*>(Y + (size_t)row * ldy + ncol) = o;
      }
    }
  }
}

// Y[row, 4c..4c+3] = fp16(sum over splits, in split order) (+ bias); the
// partials are [S][M][N], Y's rows lie ldy elements apart
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ part,
                                                     const f16* __restrict__ bias,
                                                     f16* __restrict__ Y, int M, int N, int ldy,
                                                     int S) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;   // 4-column quad index
  const size_t nq = (size_t)M * (N / 4);
  if (q >= nq) return;
  const size_t off = q * 4;
  float4 s = *reinterpret_cast<const float4*>(part + off);
  for (int i = 1; i < S; ++i) {
    const float4 v = *reinterpret_cast<const float4*>(part + (size_t)i * M * N + off);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  f16x4 o;
  o.x = f32_to_f16(s.x);
  o.y = f32_to_f16(s.y);
  o.z = f32_to_f16(s.z);
  o.w = f32_to_f16(s.w);
  const size_t row = off / (size_t)N;
  const int col = (int)(off - row * (size_t)N);
  if (bias) {
    o.x = o.x + bias[col];
    o.y = o.y + bias[col + 1];
    o.z = o.z + bias[col + 2];
    o.w = o.w + bias[col + 3];
  }
  *reinterpret_cast<f16x4*>(Y + row * (size_t)ldy + col) = o;
}

template <int WAVES_M, int WAVES_N, bool G64, bool AZ>
hipError_t launch_wgz(const GemmArgs& a, int split, float* part, hipStream_t st) {
  constexpr int BM = 16 * kMT * WAVES_M;
  constexpr int BN = 16 * kNTiles * WAVES_N;
  const int tiles = ((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  const int KT = a.K / kBK;
  const int kts = (KT + split - 1) / split;
  const int nsplit = split > 1 ? (KT + kts - 1) / kts : 1;   // every split non-empty
  hipLaunchKernelGGL((occ2_kernel<WAVES_M, WAVES_N, G64, AZ>), dim3(tiles * nsplit),
                     dim3(64 * WAVES_M * WAVES_N), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                     static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), nsplit > 1 ? part : nullptr, a.M, a.N, a.K, a.G,
                     nsplit > 1 ? kts : KT, a.ldx, a.ldy);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  return launch_splitk_reduce(part, a.bias, a.y, a.M, a.N, a.ldy, nsplit, st);
}

// Zero-point form by the call (w4a16_device.h).
template <int WAVES_M, int WAVES_N, bool G64>
hipError_t launch_wg(const GemmArgs& a, int split, float* part, hipStream_t st) {
  return a.any_zeros ? launch_wgz<WAVES_M, WAVES_N, G64, true>(a, split, part, st)
                     : launch_wgz<WAVES_M, WAVES_N, G64, false>(a, split, part, st);
}

}  // namespace

bool occ2_gemm_applicable(int M, int N, int K, int G) {
  (void)M;
  return K % kBK == 0 && N % 4 == 0 && G % 32 == 0 && K % G == 0;
}

hipError_t launch_splitk_reduce(const float* part, const void* bias, void* y, int M, int N, int ldy,
                                int S, hipStream_t st) {
  const size_t nq = (size_t)M * (size_t)(N / 4);
  hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, st, part,
                     static_cast<const f16*>(bias), static_cast<f16*>(y), M, N, ldy, S);
  return hipGetLastError();
}

int occ2_splits(int K, int split) {
  const int KT = K / kBK;
  if (split <= 1 || KT <= 1) return 1;
  const int kts = (KT + split - 1) / split;
  return (KT + kts - 1) / kts;
}

size_t occ2_workspace_bytes(int M, int N, int K, int split) {
  const int s = occ2_splits(K, split);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// waves 1 x 4: 128 x 256 tiles.  split > 1: fp32 partials in `part`
// (occ2_workspace_bytes), then launch_splitk_reduce.
hipError_t launch_occ2_gemm(const GemmArgs& a, int split, float* part, hipStream_t st) {
  if (!occ2_gemm_applicable(a.M, a.N, a.K, a.G)) return hipErrorInvalidValue;
  if (occ2_splits(a.K, split) > 1 && !part) return hipErrorInvalidValue;
  return a.G % 64 == 0 ? launch_wg<1, 4, true>(a, split, part, st)
                       : launch_wg<1, 4, false>(a, split, part, st);
}

}  // namespace w4a16
