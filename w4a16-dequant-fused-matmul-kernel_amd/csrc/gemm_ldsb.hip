// Prefill W4A16 GEMM on gfx950: the weight tile dequantised once per
// workgroup into LDS, eight waves sharing it at two waves per SIMD
// (v_mfma_f32_16x16x32_f16, fp32 accumulation).
//
// Replaces the large-M regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128: fp16 dequant of the weight
// tile, tl.dot with fp32 accumulation, fp16 store).
//
// Design:
//   * a workgroup of 8 waves (4 along M x 2 along N) owns a 256 x BN tile of Y
//     (BN = 32 * NTW: 224 or 256); a wave owns 64 rows x 16*NTW columns, at most
//     128 accumulator registers, so each SIMD runs two waves;
//   * per 64-k step the workgroup stages two fp16 tiles in LDS: activations
//     A[256 rows][64 k] (each thread loads 4 octets) and the dequantised weight
//     tile B[BN columns][64 k] (each thread loads one 16-byte quad = 4 columns of
//     one packed row and dequantises it into 4 LDS slots).  Every weight is
//     dequantised once per workgroup, and the activation tile feeds BN columns;
//   * a packed int32 word holds the 8 k of one column that an MFMA lane needs:
//     dequant (magic-number packed fp16, w4a16_device.h) yields them in pair
//     order (0,4,1,5,2,6,3,7); activation octets are permuted the same way;
//   * LDS rows padded to 144 bytes (16-lane fragment reads hit distinct banks),
//     both tiles double-buffered, one barrier per k-step; global loads run one
//     step ahead in registers;
//   * 224-column tiles give N = 14336 exactly 64 column tiles, so the C4 shape
//     fills four whole rounds of 256 workgroups;
//   * XCD-aware grouped tile order; epilogue: fp16 RNE, optional fp16 bias add
//     (W4A16Linear's `y + bias`, linear.py:90-91).
// Requirements (checked by the caller): K % 64 == 0, N % 4 == 0, G % 32 == 0,
// K % G == 0, 16-byte aligned x/qweight, 8-byte aligned scales/zeros, and x,
// qweight, scales, zeros each below 2 GiB.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kBK = 64;
constexpr int kLdsRow = 9;      // uint4 per LDS row: 8 octets + 1 pad
constexpr int kGroupM = 4;      // M-tiles per group of the tile order
constexpr int kWavesM = 4, kWavesN = 2;
constexpr int kNT = 64 * kWavesM * kWavesN;   // 512 threads
constexpr int kMTW = 4;                       // 16-row MFMA tiles per wave (64 rows)
constexpr int kBM = 16 * kMTW * kWavesM;      // 256
constexpr int kAPerT = kBM * 8 / kNT;         // activation octets per thread (4)

template <int NTW>
__global__ __launch_bounds__(kNT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void ldsb_kernel(const f16* __restrict__ X, const uint32_t* __restrict__ QW,
                 const uint16_t* __restrict__ SC, const uint16_t* __restrict__ ZR,
                 const f16* __restrict__ bias, f16* __restrict__ Y, int M, int N, int K, int G,
                 int ldx, int ldy) {
  constexpr int BNW = 16 * NTW;             // columns per wave
  constexpr int BN = BNW * kWavesN;         // columns per workgroup
  constexpr int QPR = BN / 4;               // weight quads per packed row
  constexpr int NQ = 8 * QPR;               // weight quads per k-step
  static_assert(NQ <= kNT, "one weight quad per thread");
  __shared__ uint4 As[2][kBM * kLdsRow];
  __shared__ uint4 Bs[2][BN * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / kWavesN;
  const int wn = wave % kWavesN;
  const int l16 = lane & 15;
  const int oct = lane >> 4;

  const int ntn = (N + BN - 1) / BN;
  const int ntm = (M + kBM - 1) / kBM;
  const int total = ntn * ntm;
  int T = (int)blockIdx.x;
  if ((total & 7) == 0) T = (T & 7) * (total >> 3) + (T >> 3);
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * kBM;
  const int n0 = (rem / gsz) * BN;
  const int KP = K >> 3;
  const int KT = K / kBK;
  const int NG = K / G;

  const MagicRegs mg = make_magic();
  // rows of X lie ldx elements apart; the range ends after row M - 1's K
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(M - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);

  // activation octets o = tid + i*kNT -> (row o/8, octet o%8)
  uint32_t a_off[kAPerT];
#pragma unroll
  for (int i = 0; i < kAPerT; ++i) {
    const int o = tid + i * kNT;
    const int gm = m0 + (o >> 3);
    a_off[i] = gm < M ? ((uint32_t)gm * (uint32_t)ldx + (uint32_t)(o & 7) * 8u) * 2u : kOobOffset;
  }
  // weight quad of this thread: packed row brow (0..7) of the step, columns bcol..+3
  const bool bq = tid < NQ;
  const int brow = tid / QPR;
  const int bcq = tid % QPR;
  const int bcol = n0 + 4 * bcq;
  const bool bnv = bq && bcol < N;
  const uint32_t b_off = bnv ? ((uint32_t)brow * (uint32_t)N + (uint32_t)bcol) * 4u : kOobOffset;
  const uint32_t s_off = bnv ? (uint32_t)bcol * 2u : kOobOffset;

  uint4 ra[kAPerT];
  uint4 rb;
  uint2 rsc, rzr;
  auto load = [&](int kt) {
    const uint32_t ak = uniform((uint32_t)kt * (uint32_t)(kBK * 2));
#pragma unroll
    for (int i = 0; i < kAPerT; ++i) ra[i] = buf_load16(rx, a_off[i], ak);
    rb = buf_load16(rw, b_off, uniform((uint32_t)kt * 8u * (uint32_t)N * 4u));
    // this quad's group: rows 0-3 of a step are k 0..31, rows 4-7 k 32..63
    const int g = (kt * kBK + 8 * brow) / G;
    const uint32_t so = bnv ? s_off + (uint32_t)g * (uint32_t)N * 2u : kOobOffset;
    rsc = buf_load8(rs, so, 0u);
    rzr = buf_load8(rz, so, 0u);
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kAPerT; ++i) {
      const int o = tid + i * kNT;
      As[buf][(o >> 3) * kLdsRow + (o & 7)] = perm_pairs(ra[i]);
    }
    if (bq) {
      const ColQ2 p01 = make_colq2(rsc.x, rzr.x), p23 = make_colq2(rsc.y, rzr.y);
      const ColQ cq[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
      const uint32_t words[4] = {rb.x, rb.y, rb.z, rb.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f16x2 d[4];
        dq_word_fast(words[c], cq[c], mg, d);
        Bs[buf][(4 * bcq + c) * kLdsRow + brow] =
            make_uint4(as_u32(d[0]), as_u32(d[1]), as_u32(d[2]), as_u32(d[3]));
      }
    }
  };

  f32x4 acc[kMTW][NTW];
#pragma unroll
  for (int i = 0; i < kMTW; ++i)
#pragma unroll
    for (int c = 0; c < NTW; ++c) acc[i][c] = f32x4{};

  const int arow = wm * (16 * kMTW) + l16;
  const int bcolw = wn * BNW + l16;
  auto compute = [&](int buf) {
    const uint4* A = &As[buf][arow * kLdsRow + oct];
    const uint4* B = &Bs[buf][bcolw * kLdsRow + oct];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f16x8 af[kMTW], bf[NTW];
#pragma unroll
      for (int i = 0; i < kMTW; ++i) af[i] = __builtin_bit_cast(f16x8, A[i * 16 * kLdsRow + 4 * ks]);
#pragma unroll
      for (int c = 0; c < NTW; ++c) bf[c] = __builtin_bit_cast(f16x8, B[c * 16 * kLdsRow + 4 * ks]);
#pragma unroll
      for (int i = 0; i < kMTW; ++i)
#pragma unroll
        for (int c = 0; c < NTW; ++c)
          acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[c], acc[i][c], 0, 0, 0);
    }
  };

  load(0);
  stage(0);
  __syncthreads();
  if (KT > 1) load(1);
  for (int kt = 0; kt < KT; ++kt) {
    compute(kt & 1);
    if (kt + 1 < KT) stage((kt + 1) & 1);   // step kt+1 into the other buffer
    __syncthreads();
    if (kt + 2 < KT) load(kt + 2);
  }

  // epilogue: lane holds D[4*oct + r][l16] of each 16x16 tile
#pragma unroll
  for (int c = 0; c < NTW; ++c) {
    const int col = n0 + wn * BNW + 16 * c + l16;
    if (col >= N) continue;
    const f16 bv = bias ? bias[col] : (f16)0.0f;
#pragma unroll
    for (int i = 0; i < kMTW; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * (16 * kMTW) + 16 * i + 4 * oct + r;
        if (row < M) {
          f16 y = f32_to_f16(acc[i][c][r]);
          if (bias) y = y + bv;
          Y[(size_t)row * ldy + col] = y;
        }
      }
    }
  }
}

template <int NTW>
hipError_t launch_ntw(const GemmArgs& a, hipStream_t st) {
  constexpr int BN = 32 * NTW;
  const dim3 grid(((a.N + BN - 1) / BN) * ((a.M + kBM - 1) / kBM));
  hipLaunchKernelGGL((ldsb_kernel<NTW>), grid, dim3(kNT), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                     static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  return hipGetLastError();
}

}  // namespace

bool ldsb_gemm_applicable(int M, int N, int K, int G) {
  (void)M;
  return K % kBK == 0 && N % 4 == 0 && G % 32 == 0 && K % G == 0;
}

// wide = false: 256 x 224 tiles; wide = true: 256 x 256 tiles.
hipError_t launch_ldsb_gemm(const GemmArgs& a, bool wide, hipStream_t st) {
  if (!ldsb_gemm_applicable(a.M, a.N, a.K, a.G)) return hipErrorInvalidValue;
  return wide ? launch_ntw<8>(a, st) : launch_ntw<7>(a, st);
}

}  // namespace w4a16
