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
//   * all global traffic uses buffer loads: the per-step k offset rides in an
//     SGPR, and rows past M / columns past N read as zero through the buffer
//     range check instead of branches;
//   * K advances 64 per step with three register stages in rotation (no copies)
//     and a double-buffered LDS activation tile, one barrier per step; loads are
//     issued two steps before their MFMAs;
//   * LDS rows are padded to 144 bytes so the ds_read_b128 of 16 rows x 16 B
//     hits 64 distinct banks;
//   * XCD-aware grouped tile order (see the kernel) keeps A/B tile re-reads in
//     each XCD's L2;
//   * epilogue: lane l holds 4 consecutive columns per output row, rounded to
//     fp16 (RNE) and stored as one 8-byte write; optional fp16 bias add
//     reproduces W4A16Linear's separate `y + bias` (linear.py:90-91).
// Requirements (checked by the caller): N % 4 == 0, G % 32 == 0, K % G == 0,
// 16-byte aligned x/qweight, 8-byte aligned scales/zeros/y/bias, and x, qweight,
// scales, zeros each below 2 GiB.  KTAIL handles K % 64 == 32.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

#ifndef W4A16_MFMA_INTERLEAVE
#define W4A16_MFMA_INTERLEAVE 0
#endif
#ifndef W4A16_OCC2_INTERLEAVE
#define W4A16_OCC2_INTERLEAVE 4
#endif

constexpr int kBK = 64;
constexpr int kLdsRow = 9;  // uint4 per LDS row: 8 octets + 1 pad
constexpr int kGroupM = 4;  // M-tiles per group of the tile order

template <int WMT, int WAVES_M, int WAVES_N, bool KTAIL, bool AZ>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void mfma_kernel(
    const f16* __restrict__ X, const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ bias, f16* __restrict__ Y, int M,
    int N, int K, int G, int ldx, int ldy) {
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

  // Tile order: the hardware deals workgroups to the 8 XCDs round-robin; give
  // each XCD a contiguous run of the grouped order below, so the tiles one XCD
  // holds at a time (about 32) share activation rows and weight columns through
  // that XCD's L2.  Grouped order: kGroupM M-tiles x all N-tiles per group.
  const int ntn = (N + BN - 1) / BN;
  const int ntm = (M + BM - 1) / BM;
  const int total = ntn * ntm;
  int T = (int)blockIdx.x;
  if ((total & 7) == 0) T = (T & 7) * (total >> 3) + (T >> 3);
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * BM;
  const int n0 = (rem / gsz) * BN;
  const int ncol = n0 + wn * 128 + 4 * l32;
  const bool nv = ncol < N;
  const int KP = K >> 3;
  const int KT = (K + kBK - 1) / kBK;
  const int NG = K / G;

  const MagicRegs mg = make_magic();
  // rows of X lie ldx elements apart; the range ends after row M - 1's K
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(M - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);

  // per-thread A slots (row, octet) and their byte offsets at k = 0
  uint32_t a_off[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int o = tid + i * NT;
    const int gm = m0 + (o >> 3);
    a_off[i] = gm < M ? ((uint32_t)gm * (uint32_t)ldx + (uint32_t)(o & 7) * 8u) * 2u : kOobOffset;
  }
  uint32_t b_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    b_off[s] = nv ? ((uint32_t)(2 * s + lhi) * (uint32_t)N + (uint32_t)ncol) * 4u : kOobOffset;
  const uint32_t s_off = nv ? (uint32_t)ncol * 2u : kOobOffset;

  struct Stage {
    uint4 a[A_PER_T];
    uint4 b[4];
    uint2 sc[2], zr[2];
  };

  auto load = [&](int kt, Stage& st) {
    const uint32_t ak = uniform((uint32_t)kt * (uint32_t)(kBK * 2));
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      uint32_t off = a_off[i];
      if (KTAIL && kt * kBK + ((tid + i * NT) & 7) * 8 >= K) off = kOobOffset;
      st.a[i] = buf_load16(rx, off, ak);
    }
    const uint32_t bk = uniform((uint32_t)kt * 8u * (uint32_t)N * 4u);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (!KTAIL || kt * kBK + 16 * s < K)
        st.b[s] = buf_load16(rw, b_off[s], bk);
      else
        st.b[s] = make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = min((kt * kBK + 32 * h) / G, NG - 1);
      const uint32_t gs = uniform((uint32_t)g * (uint32_t)N * 2u);
      st.sc[h] = buf_load8(rs, s_off, gs);
      st.zr[h] = buf_load8(rz, s_off, gs);
    }
  };

  auto store_a = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int o = tid + i * NT;
      As[buf][(o >> 3) * kLdsRow + (o & 7)] = perm_pairs(st.a[i]);
    }
  };

  f32x16 acc[WMT][4];
#pragma unroll
  for (int i = 0; i < WMT; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = f32x16{};

  const int arow = wm * (32 * WMT) + l32;
  // One k-step: four 16-k sub-steps.  Sub-step s+1's B dequant (VALU) and A
  // fragment reads (LDS) are issued alongside sub-step s's MFMAs; a scheduling
  // barrier between sub-steps keeps the compiler from hoisting further ahead
  // (which would raise register pressure past the 512-VGPR budget).
  auto compute = [&](const Stage& st, int buf, int kt) {
    const int nsub = (KTAIL && kt * kBK + 32 >= K) ? 2 : 4;
    ColQ cq[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const ColQ2 p01 = make_colq2<AZ>(st.sc[h].x, st.zr[h].x);
      const ColQ2 p23 = make_colq2<AZ>(st.sc[h].y, st.zr[h].y);
      cq[h][0] = colq_of<0>(p01);
      cq[h][1] = colq_of<1>(p01);
      cq[h][2] = colq_of<0>(p23);
      cq[h][3] = colq_of<1>(p23);
    }
    const uint4* A = &As[buf][arow * kLdsRow + lhi];
    auto dequant = [&](int s, f16x8 bf[4]) {
      const uint32_t words[4] = {st.b[s].x, st.b[s].y, st.b[s].z, st.b[s].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f16x2 d[4];
        dq_word_fast<AZ>(words[c], cq[s >> 1][c], mg, d);
        bf[c] = f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
      }
    };
    f16x8 af[2][WMT], bf[2][4];
#pragma unroll
    for (int mt = 0; mt < WMT; ++mt) af[0][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow]);
    dequant(0, bf[0]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s >= nsub) break;
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < nsub) {
#pragma unroll
        for (int mt = 0; mt < WMT; ++mt)
          af[nxt][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow + 2 * (s + 1)]);
        dequant(s + 1, bf[nxt]);
      }
#pragma unroll
      for (int mt = 0; mt < WMT; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[mt][c] =
              __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][mt], bf[cur][c], acc[mt][c], 0, 0, 0);
#if W4A16_MFMA_INTERLEAVE
      // Issue pattern for this sub-step: the next sub-step's fragment reads
      // first, then one MFMA followed by a few dequant VALU ops, so the VALU
      // work co-issues while the matrix core is busy.
      __builtin_amdgcn_sched_group_barrier(0x100, WMT, 0);   // DS reads
#pragma unroll
      for (int i = 0; i < 4 * WMT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, W4A16_MFMA_INTERLEAVE, 0);  // VALU
      }
#endif
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Three register stages in rotation: step kt computes from stage kt%3 while
  // step kt+2's loads fly, so each load has two k-steps to arrive.  A single
  // loop exit keeps the accumulators in one set of registers.
  Stage s0, s1, s2;
  load(0, s0);
  if (KT > 1) load(1, s1);
  store_a(s0, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 2 < KT; kt += 3) {
    // LDS buffer = step parity; a 3-step body flips it every iteration
    const int p = kt & 1;
    load(kt + 2, s2);
    compute(s0, p, kt);
    store_a(s1, p ^ 1);
    __syncthreads();
    if (kt + 3 < KT) load(kt + 3, s0);
    compute(s1, p ^ 1, kt + 1);
    store_a(s2, p);
    __syncthreads();
    if (kt + 4 < KT) load(kt + 4, s1);
    compute(s2, p, kt + 2);
    if (kt + 3 < KT) store_a(s0, p ^ 1);
    __syncthreads();
  }
  // 1 or 2 steps left: step kt in s0, its activations in LDS buffer kt % 2
  if (kt < KT) {
    const int b0 = kt & 1;
    compute(s0, b0, kt);
    if (kt + 1 < KT) {
      store_a(s1, b0 ^ 1);
      __syncthreads();
      compute(s1, b0 ^ 1, kt + 1);
    }
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
        *reinterpret_cast<f16x4*>(Y + (size_t)row * ldy + ncol) = o;
      }
    }
  }
}

// Two-waves-per-SIMD variant: each wave owns (32*WMT) rows x 64 columns (two
// columns per lane, 128 accumulator registers), so a SIMD holds two waves (from
// two workgroups) and one wave's dequant and memory waits overlap the other's
// MFMAs.  B lane l of n-tile j is column 2*(l%32) + j of the wave's 64; the
// epilogue stores 2 consecutive columns per lane.  One A register stage and two
// B register stages; K must be a multiple of 128 (two steps per iteration).
template <int WMT, int WAVES_M, int WAVES_N, bool AZ>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma_occ2_kernel(const f16* __restrict__ X, const uint32_t* __restrict__ QW,
                      const uint16_t* __restrict__ SC, const uint16_t* __restrict__ ZR,
                      const f16* __restrict__ bias, f16* __restrict__ Y, int M, int N, int K,
                      int G, int ldx, int ldy) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int BM = 32 * WMT * WAVES_M;
  constexpr int BN = 64 * WAVES_N;
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

  const int ntn = (N + BN - 1) / BN;
  const int ntm = (M + BM - 1) / BM;
  const int total = ntn * ntm;
  int T = (int)blockIdx.x;
  if ((total & 7) == 0) T = (T & 7) * (total >> 3) + (T >> 3);
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * BM;
  const int n0 = (rem / gsz) * BN;
  const int ncol = n0 + wn * 64 + 2 * l32;
  const bool nv = ncol < N;
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

  uint32_t a_off[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int o = tid + i * NT;
    const int gm = m0 + (o >> 3);
    a_off[i] = gm < M ? ((uint32_t)gm * (uint32_t)ldx + (uint32_t)(o & 7) * 8u) * 2u : kOobOffset;
  }
  const uint32_t b_off = nv ? ((uint32_t)lhi * (uint32_t)N + (uint32_t)ncol) * 4u : kOobOffset;
  const uint32_t s_off = nv ? (uint32_t)ncol * 2u : kOobOffset;

  struct StageB {
    uint2 b[4];            // k-sub s: packed row 2s + lhi, columns ncol, ncol+1
    uint32_t sc[2], zr[2];
  };
  uint4 ra[A_PER_T];

  auto load_a = [&](int kt) {
    const uint32_t ak = uniform((uint32_t)kt * (uint32_t)(kBK * 2));
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) ra[i] = buf_load16(rx, a_off[i], ak);
  };
  auto load_b = [&](int kt, StageB& st) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      st.b[s] = buf_load8(rw, b_off, uniform(((uint32_t)kt * 8u + 2u * (uint32_t)s) * (uint32_t)N * 4u));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = (kt * kBK + 32 * h) / G;
      const uint32_t gs = uniform((uint32_t)g * (uint32_t)N * 2u);
      st.sc[h] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)s_off, (int)gs, 0);
      st.zr[h] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rz, (int)s_off, (int)gs, 0);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int o = tid + i * NT;
      As[buf][(o >> 3) * kLdsRow + (o & 7)] = perm_pairs(ra[i]);
    }
  };

  f32x16 acc[WMT][2];
#pragma unroll
  for (int i = 0; i < WMT; ++i) {
    acc[i][0] = f32x16{};
    acc[i][1] = f32x16{};
  }

  const int arow = wm * (32 * WMT) + l32;
  auto compute = [&](const StageB& st, int buf) {
    ColQ cq[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const ColQ2 q2 = make_colq2<AZ>(st.sc[h], st.zr[h]);
      cq[h][0] = colq_of<0>(q2);
      cq[h][1] = colq_of<1>(q2);
    }
    const uint4* A = &As[buf][arow * kLdsRow + lhi];
    auto dequant = [&](int s, f16x8 bf[2]) {
      const uint32_t words[2] = {st.b[s].x, st.b[s].y};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f16x2 d[4];
        dq_word_fast<AZ>(words[c], cq[s >> 1][c], mg, d);
        bf[c] = f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
      }
    };
    f16x8 af[2][WMT], bf[2][2];
#pragma unroll
    for (int mt = 0; mt < WMT; ++mt) af[0][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow]);
    dequant(0, bf[0]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < 4) {
#pragma unroll
        for (int mt = 0; mt < WMT; ++mt)
          af[nxt][mt] = __builtin_bit_cast(f16x8, A[mt * 32 * kLdsRow + 2 * (s + 1)]);
        dequant(s + 1, bf[nxt]);
      }
#pragma unroll
      for (int mt = 0; mt < WMT; ++mt)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[mt][c] =
              __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][mt], bf[cur][c], acc[mt][c], 0, 0, 0);
#if W4A16_OCC2_INTERLEAVE
      __builtin_amdgcn_sched_group_barrier(0x100, WMT, 0);   // DS reads
#pragma unroll
      for (int i = 0; i < 2 * WMT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, W4A16_OCC2_INTERLEAVE, 0);  // VALU
      }
#endif
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  StageB b0, b1;
  load_a(0);
  load_b(0, b0);
  store_a(0);
  __syncthreads();
  load_a(1);
  load_b(1, b1);
  for (int kt = 0; kt < KT; kt += 2) {
    compute(b0, 0);                 // step kt
    store_a(1);                     // step kt+1
    __syncthreads();
    if (kt + 2 < KT) {
      load_a(kt + 2);
      load_b(kt + 2, b0);
    }
    compute(b1, 1);                 // step kt+1
    if (kt + 2 < KT) store_a(0);    // step kt+2
    __syncthreads();
    if (kt + 3 < KT) {
      load_a(kt + 3);
      load_b(kt + 3, b1);
    }
  }

  if (!nv) return;
  f16 bv0 = (f16)0.0f, bv1 = (f16)0.0f;
  if (bias) {
    const uint32_t b2 = *reinterpret_cast<const uint32_t*>(bias + ncol);
    bv0 = as_h(b2 & 0xFFFFu);
    bv1 = as_h(b2 >> 16);
  }
#pragma unroll
  for (int mt = 0; mt < WMT; ++mt) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int row = m0 + wm * (32 * WMT) + mt * 32 + 8 * (a >> 2) + 4 * lhi + (a & 3);
      if (row < M) {
        f16x2 o;
        o.x = f32_to_f16(acc[mt][0][a]);
        o.y = f32_to_f16(acc[mt][1][a]);
        if (bias) {
          o.x = o.x + bv0;
          o.y = o.y + bv1;
        }
        *reinterpret_cast<f16x2*>(Y + (size_t)row * ldy + ncol) = o;
      }
    }
  }
}

template <int WMT, int WAVES_M, int WAVES_N, bool AZ>
hipError_t launch_occ2(const GemmArgs& a, hipStream_t st) {
  constexpr int BM = 32 * WMT * WAVES_M;
  constexpr int BN = 64 * WAVES_N;
  dim3 grid(((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM));
  hipLaunchKernelGGL((mfma_occ2_kernel<WMT, WAVES_M, WAVES_N, AZ>), grid,
                     dim3(64 * WAVES_M * WAVES_N), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                     static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  return hipGetLastError();
}

template <int WMT, int WAVES_M, int WAVES_N, bool AZ>
hipError_t launch_cfg(const GemmArgs& a, hipStream_t st) {
  constexpr int BM = 32 * WMT * WAVES_M;
  constexpr int BN = 128 * WAVES_N;
  dim3 grid(((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM));
  dim3 block(64 * WAVES_M * WAVES_N);
  const f16* x = static_cast<const f16*>(a.x);
  const uint32_t* qw = reinterpret_cast<const uint32_t*>(a.qw);
  const uint16_t* sc = static_cast<const uint16_t*>(a.sc);
  const uint16_t* zr = static_cast<const uint16_t*>(a.zr);
  const f16* bias = static_cast<const f16*>(a.bias);
  f16* y = static_cast<f16*>(a.y);
  if (a.K % kBK == 0)
    hipLaunchKernelGGL((mfma_kernel<WMT, WAVES_M, WAVES_N, false, AZ>), grid, block, 0, st, x, qw, sc,
                       zr, bias, y, a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  else
    hipLaunchKernelGGL((mfma_kernel<WMT, WAVES_M, WAVES_N, true, AZ>), grid, block, 0, st, x, qw, sc,
                       zr, bias, y, a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  return hipGetLastError();
}

}  // namespace

// Tile configurations the planner takes (plans name them by number):
// cfg 1: 128 x 256 (2 x 2 waves, each 64 x 128), 32x32x16 MFMA
// cfg 2:  32 x 512 (4 waves along N, each 32 x 128), 32x32x16 MFMA
// cfg 6: 128 x 256, two waves per SIMD (1 x 4 waves, each 128 x 64), 32x32x16
// cfg 7: 128 x 256, two waves per SIMD, 16x16x32 MFMA (gemm_occ2.hip)
// cfg 11: 128 x 256 as cfg 7, packed weights streamed into LDS four k-steps
//         ahead (gemm_stream.hip)
// cfg 12:  32 x 256, the cfg 11 kernel with 2 m-tiles per wave (small M)
// cfg 13:  64 x 256, the cfg 11 kernel with 4 m-tiles per wave
// cfg 14: 128 x 256, the cfg 11 kernel with 8 waves in two k-slices
// Numbers 0, 3, 4, 5, 8, 9 and 10 belonged to tilings that measured slower
// on every shape and were retired; a plan naming them is refused.
MfmaTile mfma_tile(int cfg) {
  switch (cfg) {
    case 1: return {128, 256};
    case 2: return {32, 512};
    case 6: return {128, 256};
    case 7: return {128, 256};
    case 11: return {128, 256};
    case 12: return {32, 256};
    case 13: return {64, 256};
    case 14: return {128, 256};
    default: return {0, 0};
  }
}

bool mfma_cfg_splits(int cfg) { return cfg == 7 || cfg >= 11; }

bool mfma_cfg_applicable(int cfg, int M, int N, int K, int G) {
  switch (cfg) {
    case 1:
    case 2: return true;
    case 6: return K % (2 * kBK) == 0;
    case 7: return occ2_gemm_applicable(M, N, K, G);
    case 11:
    case 12:
    case 13:
    case 14: return stream_gemm_applicable(M, N, K, G);
    default: return false;
  }
}

bool operands_fit(int M, int N, int K, int G) {
  const uint64_t xb = (uint64_t)M * K * 2, wb = (uint64_t)(K / 8) * N * 4,
                 sb = (uint64_t)(K / G) * N * 2;
  return xb < (1ull << 31) && wb < (1ull << 31) && sb < (1ull << 31);
}

bool mfma_fits(int M, int N, int K, int G) { return operands_fit(M, N, K, G); }

hipError_t launch_mfma(const GemmArgs& a, int cfg, int split, float* part, hipStream_t st) {
  if (split > 1 && !mfma_cfg_splits(cfg)) return hipErrorInvalidValue;
  switch (cfg) {
    case 1:
      return a.any_zeros ? launch_cfg<2, 2, 2, true>(a, st) : launch_cfg<2, 2, 2, false>(a, st);
    case 2:
      return a.any_zeros ? launch_cfg<1, 1, 4, true>(a, st) : launch_cfg<1, 1, 4, false>(a, st);
    case 6:
      if (a.K % (2 * kBK) != 0) return hipErrorInvalidValue;
      return a.any_zeros ? launch_occ2<4, 1, 4, true>(a, st) : launch_occ2<4, 1, 4, false>(a, st);
    case 7: return launch_occ2_gemm(a, split, part, st);
    case 11: return launch_stream_gemm(a, 128, split, part, st);
    case 12: return launch_stream_gemm(a, 32, split, part, st);
    case 13: return launch_stream_gemm(a, 64, split, part, st);
    case 14: return launch_stream_gemm(a, 128, split, part, st, 2);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
