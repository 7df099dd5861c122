// Prefill W4A16 GEMM on gfx950 matrix cores with the weight tile dequantised
// once per workgroup into LDS (v_mfma_f32_32x32x16_f16, fp32 accumulation).
//
// Replaces the large-M regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128: fp16 dequant of the weight
// tile, tl.dot with fp32 accumulation, fp16 store).
//
// Design:
//   * a workgroup of 2 x 2 waves owns a 256 x 256 tile of Y; each wave owns
//     128 x 128 (4 x 4 MFMA tiles, 256 accumulator registers);
//   * per 64-k step the workgroup stages two fp16 tiles in LDS: activations
//     A[256 rows][64 k] and dequantised weights B[256 columns][64 k].  Each
//     thread dequantises 8 packed words (64 weights) -- 1.6 VALU per MFMA,
//     where dequantising per wave in registers costs twice that;
//   * a packed int32 word holds the 8 k of one column that an MFMA lane needs:
//     it is dequantised (magic-number packed fp16, w4a16_device.h) straight into
//     one 16-byte LDS slot.  Dequant yields k in pair order (0,4,1,5,2,6,3,7);
//     activation octets are permuted the same way, so A and B agree on k;
//   * B rows in LDS are the columns in "interleave by 4" order inside each
//     wave's 128 columns: MFMA n-tile t, lane column j holds column 4j + t.  So
//     the 16-lane fragment reads walk consecutive 144-byte LDS rows (no bank
//     conflicts) and in the epilogue each lane owns 4 consecutive columns of a
//     row (one 8-byte store);
//   * LDS rows are padded to 144 bytes; A and B are double-buffered (144 KiB);
//     one barrier per k-step;
//   * global loads run two k-steps ahead (two register stages in alternation);
//     rows past M / columns past N read as zero through the buffer range check;
//   * XCD-aware grouped tile order as in the register-B kernel;
//   * epilogue: fp16 RNE, optional fp16 bias add (W4A16Linear's `y + bias`,
//     linear.py:90-91).
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
constexpr int kWavesM = 2, kWavesN = 2;
constexpr int kNT = 64 * kWavesM * kWavesN;
constexpr int kWMT = 4, kWNT = 4;                 // 32x32 MFMA tiles per wave
constexpr int kBM = 32 * kWMT * kWavesM;          // 256
constexpr int kBN = 32 * kWNT * kWavesN;          // 256
constexpr int kAPerT = kBM * 8 / kNT;             // A octets per thread per step (8)
constexpr int kBQuads = 8 * kBN / 4;              // packed uint4 per step (512)
constexpr int kBPerT = kBQuads / kNT;             // 2
static_assert(kBQuads % kNT == 0 && (kBM * 8) % kNT == 0, "even split");
static_assert(kBN / 4 == 64, "one packed row of the tile per wave-load");

// LDS row of column j (0 <= j < kBN) of the B tile: interleave by 4 inside
// each wave's 128 columns.
__device__ __forceinline__ int b_row(int j) {
  const int w = j >> 7, jj = j & 127;
  return (w << 7) + ((jj & 3) << 5) + (jj >> 2);
}

__global__ __launch_bounds__(kNT) void lds_kernel(const f16* __restrict__ X,
                                                  const uint32_t* __restrict__ QW,
                                                  const uint16_t* __restrict__ SC,
                                                  const uint16_t* __restrict__ ZR,
                                                  const f16* __restrict__ bias,
                                                  f16* __restrict__ Y, int M, int N, int K,
                                                  int G, int ldx, int ldy) {
  __shared__ uint4 As[2][kBM * kLdsRow];
  __shared__ uint4 Bs[2][kBN * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / kWavesN;
  const int wn = wave % kWavesN;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;

  // Tile order (see the register-B kernel): each XCD takes a contiguous run of
  // a grouped order, kGroupM M-tiles x all N-tiles per group.
  const int ntn = (N + kBN - 1) / kBN;
  const int ntm = (M + kBM - 1) / kBM;
  const int total = ntn * ntm;
  int T = (int)blockIdx.x;
  if ((total & 7) == 0) T = (T & 7) * (total >> 3) + (T >> 3);
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * kBM;
  const int n0 = (rem / gsz) * kBN;
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

  // A slots: octet o = tid + i*kNT -> (row o/8, octet o%8) of the 256 x 64 tile.
  uint32_t a_off[kAPerT];
#pragma unroll
  for (int i = 0; i < kAPerT; ++i) {
    const int o = tid + i * kNT;
    const int gm = m0 + (o >> 3);
    a_off[i] = gm < M ? ((uint32_t)gm * (uint32_t)ldx + (uint32_t)(o & 7) * 8u) * 2u : kOobOffset;
  }
  // B slots: quad q = tid + i*kNT -> packed row q/64 (wave-uniform), columns
  // n0 + 4*(q%64) .. +3.  Slot i = 0 covers packed rows 0-3, i = 1 rows 4-7.
  const int bq = lane;                       // column quad within the tile
  const int bcol = n0 + 4 * bq;
  const bool bnv = bcol < N;
  const uint32_t b_voff = bnv ? (uint32_t)bcol * 4u : kOobOffset;
  const uint32_t s_voff = bnv ? (uint32_t)bcol * 2u : kOobOffset;
  const int prow0 = wave;                    // packed row of slot 0 (slot 1: +4)

  struct Stage {
    uint4 a[kAPerT];
    uint4 b[kBPerT];
    uint2 s[kBPerT], z[kBPerT];
  };

  auto load = [&](int kt, Stage& st) {
    const uint32_t ak = uniform((uint32_t)kt * (uint32_t)(kBK * 2));
#pragma unroll
    for (int i = 0; i < kAPerT; ++i) st.a[i] = buf_load16(rx, a_off[i], ak);
#pragma unroll
    for (int i = 0; i < kBPerT; ++i) {
      const int prow = prow0 + 4 * i;
      const uint32_t bk = uniform(((uint32_t)kt * 8u + (uint32_t)prow) * (uint32_t)N * 4u);
      st.b[i] = buf_load16(rw, b_voff, bk);
      // rows 0-3 of the step are k 0..31 (one group), rows 4-7 k 32..63
      const int g = (kt * kBK + 32 * i) / G;
      const uint32_t gs = uniform((uint32_t)g * (uint32_t)N * 2u);
      st.s[i] = buf_load8(rs, s_voff, gs);
      st.z[i] = buf_load8(rz, s_voff, gs);
    }
  };

  // Dequantise the B quads into LDS and write the permuted activation octets.
  auto stage = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < kBPerT; ++i) {
      const int prow = prow0 + 4 * i;
      const ColQ2 p01 = make_colq2(st.s[i].x, st.z[i].x), p23 = make_colq2(st.s[i].y, st.z[i].y);
      const ColQ cq[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
      const uint32_t words[4] = {st.b[i].x, st.b[i].y, st.b[i].z, st.b[i].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f16x2 d[4];
        dq_word_fast(words[c], cq[c], mg, d);
        uint4 v;
        v.x = as_u32(d[0]);
        v.y = as_u32(d[1]);
        v.z = as_u32(d[2]);
        v.w = as_u32(d[3]);
        Bs[buf][b_row(4 * bq + c) * kLdsRow + prow] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < kAPerT; ++i) {
      const int o = tid + i * kNT;
      As[buf][(o >> 3) * kLdsRow + (o & 7)] = perm_pairs(st.a[i]);
    }
  };

  f32x16 acc[kWMT][kWNT];
#pragma unroll
  for (int i = 0; i < kWMT; ++i)
#pragma unroll
    for (int j = 0; j < kWNT; ++j) acc[i][j] = f32x16{};

  const int arow = wm * (32 * kWMT) + l32;
  const int brow = wn * (32 * kWNT) + l32;
  auto compute = [&](int buf) {
    const uint4* A = &As[buf][arow * kLdsRow + lhi];
    const uint4* B = &Bs[buf][brow * kLdsRow + lhi];
    f16x8 af[2][kWMT], bf[2][kWNT];
#pragma unroll
    for (int mt = 0; mt < kWMT; ++mt) af[0][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow]);
#pragma unroll
    for (int nt = 0; nt < kWNT; ++nt) bf[0][nt] = __builtin_bit_cast(f16x8, B[nt * 32 * kLdsRow]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < 4) {
#pragma unroll
        for (int mt = 0; mt < kWMT; ++mt)
          af[nxt][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow + 2 * (s + 1)]);
#pragma unroll
        for (int nt = 0; nt < kWNT; ++nt)
          bf[nxt][nt] = __builtin_bit_cast(f16x8, B[nt * 32 * kLdsRow + 2 * (s + 1)]);
      }
#pragma unroll
      for (int mt = 0; mt < kWMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kWNT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][mt], bf[cur][nt],
                                                               acc[mt][nt], 0, 0, 0);
    }
  };

  // Two register stages in alternation: during step kt the registers hold the
  // global data of steps kt+1 (staged into LDS this step) and kt+2 (in flight).
  Stage r0, r1;
  load(0, r0);
  if (KT > 1) load(1, r1);
  stage(r0, 0);
  if (KT > 2) load(2, r0);
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    // step kt: LDS buffer 0 (kt even); stage step kt+1 (r1) into buffer 1
    compute(0);
    stage(r1, 1);
    if (kt + 3 < KT) load(kt + 3, r1);
    __syncthreads();
    // step kt+1: buffer 1; stage step kt+2 (r0) into buffer 0
    compute(1);
    if (kt + 2 < KT) {
      stage(r0, 0);
      if (kt + 4 < KT) load(kt + 4, r0);
    }
    __syncthreads();
  }
  if (kt < KT) compute(0);   // odd KT: the last step sits in buffer 0

  const int ncol = n0 + wn * (32 * kWNT) + 4 * l32;
  if (ncol >= N) return;
  f16 bv[4] = {(f16)0.0f, (f16)0.0f, (f16)0.0f, (f16)0.0f};
  if (bias) {
    const uint2 b2 = *reinterpret_cast<const uint2*>(bias + ncol);
    bv[0] = as_h(b2.x & 0xFFFFu);
    bv[1] = as_h(b2.x >> 16);
    bv[2] = as_h(b2.y & 0xFFFFu);
    bv[3] = as_h(b2.y >> 16);
  }
#pragma unroll
  for (int mt = 0; mt < kWMT; ++mt) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int row = m0 + wm * (32 * kWMT) + mt * 32 + 8 * (a >> 2) + 4 * lhi + (a & 3);
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
        *reinterpret_cast<f16x4*>(Y + (size_t)row * ldy + ncol) = o;
      }
    }
  }
}

}  // namespace

bool lds_gemm_applicable(int M, int N, int K, int G) {
  (void)M;
  return K % kBK == 0 && N % 4 == 0 && G % 32 == 0 && K % G == 0;
}

hipError_t launch_lds_gemm(const GemmArgs& a, hipStream_t st) {
  const int tiles = ((a.N + kBN - 1) / kBN) * ((a.M + kBM - 1) / kBM);
  hipLaunchKernelGGL(lds_kernel, dim3(tiles), dim3(kNT), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                     static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  return hipGetLastError();
}

}  // namespace w4a16
