// Decode GEMV for small M (M <= 8): Y = X @ dequant(qweight) streamed from HBM.
//
// Replaces the decode regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128 at M = 1..16, BLOCK_M >= 16).
//
// Layout of the work (both kernels):
//   * a workgroup (WAVES waves) owns a block of CW = 4*CWL consecutive columns
//     (16, 32, 64, 128 or 256); in a wave, CWL lanes cover one packed row (one
//     dwordx4 = 4 columns per lane) and the wave's 64/CWL row-lanes sit on
//     different packed rows;
//   * dequant is the packed-fp16 magic-number form (w4a16_device.h); the dot
//     product is v_dot2_f32_f16 with fp32 accumulation, or (staged kernel,
//     64-column blocks, M <= 2, cfg 6 / 7) v_mfma_f32_16x16x32_f16 with the
//     activations broadcast over its m-rows;
//     weights are read with the non-temporal hint: each byte is used once;
//   * reduction over row-lanes: DPP row rotations and a permlane
//     transpose-reduce inside the wave (two permlane32 swaps for 128-column
//     blocks), then the waves in order through LDS -- deterministic
//     (gemv_reduce_store);
//   * at most two register batches per lane are in flight: a third (loads two
//     batches ahead) measured 3-23 % slower on every multi-batch shape, its
//     registers costing a workgroup per CU (M = 1, K = 4096, N = 28672 16.4 ->
//     20.2 us on 64-column blocks, 15.5 -> 16.2 on 128-column blocks);
//   * workgroup -> column block is XCD-aware: the hardware deals workgroups to the
//     8 XCDs round-robin, and consecutive column blocks are given to the same XCD
//     so that neighbouring row segments share that XCD's L2 lines (measured on
//     MI355X: ~1 us per C2 call against the identity order, where both halves of
//     a 128-byte line are fetched by two XCDs);
//   * split-K where the column blocks cannot fill the CUs and K is long (the
//     planner's rule; a plan can also force it): each workgroup writes fp32
//     partials and a second kernel sums the splits in split order
//     (deterministic).
// gemv_direct_kernel (M <= 2, activations read directly: the whole X is a few
// KiB and stays in L2, and no barrier stands before the first dot product):
// the rows are dealt to the row-lanes in sweeps, so each batch is one
// contiguous run of rows and a lane's first rows are the first to arrive.
// gemv_kernel (M > 2, or M <= 2 with X staged in LDS): a row-lane's rows come
// in batches of BR rows (4 with 8 waves, 2 with 16) aligned to absolute
// multiples of BR, so a 4-row half (32 k, G % 32 == 0) lies in one group and a
// batch needs one scale / zero load per half; for M <= 2 the batches are dealt
// to the row-lanes in sweeps (batch i of every row-lane together is one
// contiguous run of rows), for M > 2 each row-lane owns a contiguous run of
// batches; every load of batch i+1 is issued before batch i is consumed; X is
// staged once per chunk in LDS, permuted to the dequantiser's pair order.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kXsEntries = 2048;          // LDS activation slots (16 B each): 32 KiB
constexpr int kNonTemporal = 2;           // buffer-load cache policy: nt

template <int WAVES>
struct GemvShape {
  static constexpr int kThreads = 64 * WAVES;
  // packed rows per batch: fewer rows per lane as the wave count grows
  static constexpr int kBatch = WAVES >= 16 ? 2 : 4;
};

// Sum the lanes' partial dot products over the workgroup's row-lanes in a
// fixed order and write y (S == 1, fp16 RNE, optional fp16 bias add) or this
// k-split's fp32 partials.  Inside each 16-lane DPP row the lanes with equal
// column quad are combined by row rotations, then a transpose-reduce over the
// wave's four 16-lane rows leaves column slot c of the lane's quad in row c
// (register-to-register, fixed order); the per-wave sums go through LDS once
// and thread t < CW adds the WAVES partial sets of its column in wave order.
template <int MT, int CWL, int WAVES>
__device__ __forceinline__ void gemv_sum_waves_store(float (&red)[WAVES][MT][4 * CWL], int tid,
                                                     int cb, int sk, int S, int N, int ldy,
                                                     const f16* __restrict__ bias,
                                                     f16* __restrict__ Y, float* __restrict__ part);

template <int MT, int CWL, int WAVES>
__device__ __forceinline__ void gemv_reduce_store(float (&acc)[MT][4],
                                                  float (&red)[WAVES][MT][4 * CWL], int tid,
                                                  int cb, int sk, int S, int N, int ldy,
                                                  const f16* __restrict__ bias, f16* __restrict__ Y,
                                                  float* __restrict__ part) {
  constexpr int CW = 4 * CWL;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cq = lane % CWL;
  if constexpr (CWL <= 16) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c] = acc[m][c];
        if constexpr (CWL <= 4) v[c] += dpp_row_ror<4>(v[c]);
        if constexpr (CWL <= 8) v[c] += dpp_row_ror<8>(v[c]);
      }
      const float r = fold_rows4(v[0], v[1], v[2], v[3]);
      if ((lane & 15) < CWL) red[wave][m][4 * cq + (lane >> 4)] = r;
    }
  } else if constexpr (CWL == 32) {
    // the wave's two halves hold the same 32 column quads (two row-lanes):
    // after the swaps the lower half holds columns 0 and 2 of each quad summed
    // over both halves, the upper half columns 1 and 3
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v0 = acc[m][0], v1 = acc[m][1], v2 = acc[m][2], v3 = acc[m][3];
      permlane32_swap(v0, v1);
      permlane32_swap(v2, v3);
      const int hi = lane >> 5;
      red[wave][m][4 * cq + hi] = v0 + v1;
      red[wave][m][4 * cq + 2 + hi] = v2 + v3;
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m)
      *reinterpret_cast<float4*>(&red[wave][m][4 * cq]) =
          make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
  }
  __syncthreads();
  gemv_sum_waves_store<MT, CWL, WAVES>(red, tid, cb, sk, S, N, ldy, bias, Y, part);
}

// Second half of the reduction (after the barrier): thread t < CW adds the
// WAVES partial sets of column t in wave order and writes y (S == 1: fp16 RNE,
// optional fp16 bias) or this k-split's fp32 partials.
template <int MT, int CWL, int WAVES>
__device__ __forceinline__ void gemv_sum_waves_store(float (&red)[WAVES][MT][4 * CWL], int tid,
                                                     int cb, int sk, int S, int N, int ldy,
                                                     const f16* __restrict__ bias,
                                                     f16* __restrict__ Y, float* __restrict__ part) {
  constexpr int CW = 4 * CWL;
  const int t = tid;
  const int col = cb * CW + t;
  const bool cv = (t < CW) && (col < N);
  float v[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float sum = 0.0f;
    if (t < CW) {
      sum = red[0][m][t];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum += red[w][m][t];
    }
    v[m] = sum;
  }

  if (S == 1) {
    if (cv) {
      const f16 b = bias ? bias[col] : (f16)0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        f16 y = f32_to_f16(v[m]);
        if (bias) y = y + b;
        Y[(size_t)m * ldy + col] = y;
      }
    }
    return;
  }

  // split-K: fp32 partials [split][M][N]; a second kernel sums the splits
  if (cv) {
#pragma unroll
    for (int m = 0; m < MT; ++m) part[((size_t)sk * MT + m) * N + col] = v[m];
  }
}

// Arguments: the first fourteen SGPRs' worth (preloaded by the dispatch, as for
// gemv_direct_kernel) are what the first loads need; the grid size is
// nblk * S, computed rather than read from the dispatch packet.
template <int MT, int CWL, int WAVES, bool STAGE, bool MF, int QPL, bool AZ>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(
    const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ X, int N, int K, int rows_per_wg,
    int S, uint32_t gmagic, int gshift, int ldx, int ldy, const f16* __restrict__ bias,
    f16* __restrict__ Y, float* __restrict__ part) {
  constexpr int kThreads = GemvShape<WAVES>::kThreads;
  constexpr int BR = GemvShape<WAVES>::kBatch;
  constexpr int RH = BR < 4 ? BR : 4;      // rows per half (a half lies in one group)
  constexpr int H = BR / RH;               // halves per batch
  // M <= 2 without staging runs gemv_direct_kernel; here X is staged in LDS
  static_assert(MT > 2 || STAGE, "M <= 2 with direct activations is gemv_direct_kernel");
  // MF: the dot products on the matrix cores (v_mfma_f32_16x16x32_f16).  With
  // 16 lanes per packed row (64-column blocks) a wave's lanes are 16 column
  // quads x 4 row-lanes, which is the MFMA's B layout (lane l: n = l % 16,
  // k-octet l / 16) with word t of the quad as n-tile t; each lane's
  // activation octet (its own row, from LDS) is the A operand, the same in all
  // 16 m-rows for M = 1 (row 1 in m-row 1 for M = 2), so the MFMA sums over
  // the wave's four row-lanes and leaves y in every m-row.  Rows past a lane's
  // run add zeros (kBranchFree), so every lane can take part in every MFMA.
  // Measured on MI355X (cfg 7: 8 waves; 144 registers, one workgroup per CU)
  // against the dot2 form of the same blocks: M = 2, K = 8192, N = 28672 32.9
  // -> 26.8 us; M = 1, K = 4096, N = 16384 9.9 -> 9.5; K = 8192, N = 16384
  // 15.5 -> 15.0.  Capped at 128 registers (two workgroups per CU) it spilled
  // and ran 15-20 % slower.
  // QPL = 2 (MF only): each lane also takes the column quad 64 columns on,
  // so a workgroup owns 128 columns with the same lane layout (two loads of
  // 256 contiguous bytes per packed row and wave instead of one of 512).
  static_assert(!MF || (CWL == 16 && MT <= 2), "MFMA dot products: 64-column layout, M <= 2");
  static_assert(QPL == 1 || (MF && QPL == 2), "two column quads per lane: MFMA form only");
  constexpr int RW = 64 / CWL;             // row-lanes per wave
  constexpr int RL = WAVES * RW;           // row-lanes per workgroup
  constexpr int CW = 4 * CWL * QPL;        // columns per workgroup
  constexpr int HW = 4 * CWL;              // columns between a lane's quads
  constexpr int CHUNK = kXsEntries / MT / BR * BR;   // packed rows of X per stage
  static_assert(CHUNK % BR == 0, "chunk must hold whole batches");
  // M <= 2 on 64-column and wider blocks: every row of a batch is processed
  // without a range check.  The end of the lane's rows `le` (the chunk's end
  // for M <= 2, below) is a multiple of the batch (K % 32 == 0, splits and
  // chunks in whole batches), so a batch is wholly inside or wholly past it,
  // and a batch past it loads zero words, scales and zeros (out-of-range
  // offsets): its weights dequantise to exactly 0, and its rows read BR zero
  // rows of X (so 0 * x never meets an inf or NaN of another row; an odd
  // number of batches above one also processes the batch after the last,
  // which lies past the chunk's end).  The batch's first row picks its LDS
  // rows, so each row's read keeps the row offset in the instruction's
  // immediate.  The per-row branch had put every
  // row's dequant under an exec mask and the next batch's loads between them:
  // measured on MI355X without it, M = 1, K = 8192, N = 28672 on 128-column
  // blocks 27.0 -> 25.6 us, K = 4096 16.0 -> 15.4, M = 2 30.2 -> 29.2, N = 16384
  // on 64-column blocks 10.4 -> 9.8; on 16-column blocks (never staged by the
  // planner) it measured slower.  XS: per m, CHUNK staged rows and BR zero rows.
  constexpr bool kBranchFree = MT <= 2 && CWL >= 16;
  constexpr int XS = kBranchFree ? CHUNK + BR : CHUNK;
  __shared__ uint4 xs[MT * XS];
  __shared__ float red[WAVES][MT][CW];

  const int nblk = (N + CW - 1) / CW;
  const int nb = nblk * S;

  // XCD-aware block order (see header comment).
  int lin = (int)blockIdx.x;
  if ((nb & 7) == 0) lin = (lin & 7) * (nb >> 3) + (lin >> 3);
  // without a split the block index is the column block (no division)
  const int cb = S == 1 ? lin : lin % nblk;
  const int sk = S == 1 ? 0 : lin / nblk;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cq = lane % CWL;
  const int rl = wave * RW + lane / CWL;
  const int n = cb * CW + 4 * cq;            // the lane's first column quad
  const int KP = K >> 3;
  // k / G for 0 <= k < 2^31 without a division in front of the first loads:
  // (umulhi(k, gmagic) + k) >> gshift with gshift = ceil(log2 G) and gmagic =
  // floor(2^32 (2^gshift - G) / G) + 1 (exact for k < 2^31; 1 for a power of two)
  auto group_of = [&](int k) {
    return (int)((__umulhi((uint32_t)k, gmagic) + (uint32_t)k) >> gshift);
  };
  const int NG = group_of(K);
  const int rb = sk * rows_per_wg;
  const int re = min(KP, rb + rows_per_wg);
  const MagicRegs mg = make_magic();
  // rows of X lie ldx elements apart; the range ends after row MT - 1's K
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(MT - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);
  const uint32_t row_bytes = (uint32_t)N * 4u;
  const uint32_t s_voff = (uint32_t)n * 2u;

  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;
  f32x4 macc[QPL][4];
#pragma unroll
  for (int q = 0; q < QPL; ++q)
#pragma unroll
    for (int c = 0; c < 4; ++c) macc[q][c] = f32x4{};
  // MF, M = 2: m-row 1 of the A operand (lanes with lane % 16 == 1) is x row 1
  const int xrow = (MF && MT == 2 && (lane & 15) == 1) ? 1 : 0;

  struct Batch {
    uint2 s[H][QPL], z[H][QPL];
    uint4 w[BR][QPL];
  };
  // Rows r0..r0+BR-1 of this lane's rows, which end at `le`.  Row u rides in
  // the SGPR offset; weight rows at or past `le` read as zero.
  auto load_batch = [&](int r0, int le, Batch& b) {
#pragma unroll
    for (int h = 0; h < H; ++h) {
      // the group differs between row-lanes: its offset goes in the VGPR operand
      const int g = min(group_of((r0 + RH * h) * 8), NG - 1);
#pragma unroll
      for (int q = 0; q < QPL; ++q) {
        // a batch past the lane's rows (issued only to keep the loads the same
        // on every path) reads nothing from memory
        const bool v = n + HW * q < N && r0 < le;
        const uint32_t so =
            v ? s_voff + (uint32_t)(HW * q) * 2u + (uint32_t)g * (uint32_t)N * 2u : kOobOffset;
        b.s[h][q] = buf_load8(rs, so, 0u);
        b.z[h][q] = buf_load8(rz, so, 0u);
      }
    }
    // One path for full and partial batches (a lane-dependent branch here would
    // move the row offset out of the SGPR and serialise the loads).
#pragma unroll
    for (int q = 0; q < QPL; ++q) {
      const uint32_t base = n + HW * q < N
                                ? ((uint32_t)r0 * (uint32_t)N + (uint32_t)(n + HW * q)) * 4u
                                : kOobOffset;
#pragma unroll
      for (int u = 0; u < BR; ++u)
        b.w[u][q] = buf_load16<kNonTemporal>(rw, r0 + u < le ? base : kOobOffset,
                                             uniform((uint32_t)u * row_bytes));
    }
  };

  auto process = [&](const Batch& b, int r0, int le, int c0) {
    // LDS row of the batch's first row: the zero rows for a batch past `le`
    const int xb = kBranchFree && r0 >= le ? CHUNK : r0 - c0;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      if constexpr (MF) {
#pragma unroll
        for (int q = 0; q < QPL; ++q) {
          const ColQ2 p01 = make_colq2<AZ>(b.s[h][q].x, b.z[h][q].x);
          const ColQ2 p23 = make_colq2<AZ>(b.s[h][q].y, b.z[h][q].y);
          const ColQ cq4[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
#pragma unroll
          for (int uu = 0; uu < RH; ++uu) {
            const int u = h * RH + uu;

            f16x2 d[4][4];
            dq_word_fast<AZ>(b.w[u][q].x, cq4[0], mg, d[0]);
            dq_word_fast<AZ>(b.w[u][q].y, cq4[1], mg, d[1]);
            dq_word_fast<AZ>(b.w[u][q].z, cq4[2], mg, d[2]);
            dq_word_fast<AZ>(b.w[u][q].w, cq4[3], mg, d[3]);
            // both operands in pair order: (w0 w4 w1 w5 w2 w6 w3 w7) against
            // the activations permuted the same way when they were staged
            const uint4 xp = xs[xrow * XS + xb + u];
#pragma unroll
            for (int c = 0; c < 4; ++c)
              macc[q][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  __builtin_bit_cast(f16x8, xp),
                  f16x8{d[c][0].x, d[c][0].y, d[c][1].x, d[c][1].y, d[c][2].x, d[c][2].y,
                        d[c][3].x, d[c][3].y},
                  macc[q][c], 0, 0, 0);
          }
        }
        continue;
      }
      const ColQ2 p01 = make_colq2<AZ>(b.s[h][0].x, b.z[h][0].x);
      const ColQ2 p23 = make_colq2<AZ>(b.s[h][0].y, b.z[h][0].y);
      const ColQ cq4[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
#pragma unroll
      for (int uu = 0; uu < RH; ++uu) {
        const int u = h * RH + uu;
        const int r = r0 + u;
        if (!kBranchFree && r >= le) break;
        f16x2 d[4][4];
        dq_word_fast<AZ>(b.w[u][0].x, cq4[0], mg, d[0]);
        dq_word_fast<AZ>(b.w[u][0].y, cq4[1], mg, d[1]);
        dq_word_fast<AZ>(b.w[u][0].z, cq4[2], mg, d[2]);
        dq_word_fast<AZ>(b.w[u][0].w, cq4[3], mg, d[3]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const uint4 xp = xs[m * XS + xb + u];
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
  };

  for (int c0 = rb; c0 < re; c0 += CHUNK) {
    const int c1 = min(re, c0 + CHUNK);
    const int nr = c1 - c0;
    // this row-lane's rows in the chunk: BR-row aligned run
    // M <= 2: batch i of row-lane rl holds rows c0 + (i RL + rl) BR .. + BR,
    // so each batch index is one contiguous run of RL * BR rows read by the
    // whole workgroup at once, and the rows of the chunk arrive in the order
    // the lanes consume them.  Measured on MI355X against contiguous runs of
    // rows per lane (cold weights, same run, µs): M = 1, K = 8192, N = 16384,
    // 64-column MFMA-dot blocks 14.9 -> 14.1, 128-column 24.5 -> 22.4; M = 2,
    // K = 8192, N = 28672, 128-column MFMA-dot 25.5 -> 24.3; M = 1, K = 4096,
    // N = 16384, 64-column 9.3 -> 8.6; within +-1.5 % on the 128- / 256-column
    // dot2 blocks.  M > 2 keeps a BR-aligned contiguous run per row-lane.
    const int per = ((nr + RL - 1) / RL + BR - 1) / BR * BR;
    constexpr bool kSweep = MT <= 2;
    const int lb = kSweep ? c0 + rl * BR : min(c1, c0 + rl * per);
    const int le = kSweep ? c1 : min(c1, lb + per);
    const int bstep = kSweep ? RL * BR : BR;     // rows from one batch to the next

    Batch ba, bb;
    {
      // Stage X rows [c0, c1) into LDS; its loads go out before the first
      // weight batch, so the barrier waits only for them.
      if (c0 != rb) __syncthreads();   // previous chunk's readers are done
      constexpr int XPT = (MT * CHUNK + kThreads - 1) / kThreads;
      uint4 xv[XPT];
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int idx = tid + i * kThreads;
        const int m = idx / CHUNK, r = idx % CHUNK;
        const uint32_t off = (m < MT && r < nr)
                                 ? ((uint32_t)m * (uint32_t)ldx + (uint32_t)(c0 + r) * 8u) * 2u
                                 : kOobOffset;
        xv[i] = buf_load16(rx, off, 0u);
      }
      // Unconditional (a lane without rows reads only out-of-range weight rows
      // and a clamped group), so the loads in flight are the same on every
      // path and the waits below count exactly; the scheduling barrier keeps
      // the activation permutes, and their waits, behind the weight loads.
      load_batch(lb, le, ba);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int idx = tid + i * kThreads;
        if (idx < MT * CHUNK) xs[(idx / CHUNK) * XS + idx % CHUNK] = perm_pairs(xv[i]);
      }
      if constexpr (XS > CHUNK) {
        if (tid < MT * BR) xs[(tid / BR) * XS + CHUNK + tid % BR] = make_uint4(0u, 0u, 0u, 0u);
      }
      __syncthreads();
    }

    // Two register batches used ping-pong.  M <= 2: the trip count is the same
    // for every lane (`per` rows; past its own run a lane's loads read nothing
    // and process() skips its rows or, branch-free, adds their zeros), and the
    // loads are unconditional, so every
    // path has the same loads in flight and the compiler's waits count
    // exactly (with lane-dependent branches around the loads, its waits at the
    // joins covered the next batch too: 2-10 % slower on multi-batch runs); a
    // one-batch run (C2) has nothing to prefetch and skips the loop.  M > 2
    // keeps the per-lane loop, which measured 6-7 % faster there (M = 3, 4,
    // K = 4096, N = 28672).
    if constexpr (MT <= 2) {
      const int nbat = (nr + RL * BR - 1) / (RL * BR);
      if (nbat == 1) {
        process(ba, lb, le, c0);
      } else {
        for (int i = 0; i < nbat; i += 2) {
          const int r0 = lb + i * bstep;
          load_batch(r0 + bstep, le, bb);
          process(ba, r0, le, c0);
          load_batch(r0 + 2 * bstep, le, ba);
          process(bb, r0 + bstep, le, c0);
        }
      }
    } else {
      for (int r0 = lb; r0 < le; r0 += 2 * BR) {
        if (r0 + BR < le) load_batch(r0 + BR, le, bb);
        process(ba, r0, le, c0);
        if (r0 + BR >= le) break;
        if (r0 + 2 * BR < le) load_batch(r0 + 2 * BR, le, ba);
        process(bb, r0 + BR, le, c0);
      }
    }
  }

  if constexpr (MF) {
    // lanes 0..15 hold column quad `lane` (all m-rows alike, m-row m = y row m
    // in component m): one partial set per wave into LDS, then the waves in order
    if (lane < 16) {
#pragma unroll
      for (int q = 0; q < QPL; ++q)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int c = 0; c < 4; ++c) red[wave][m][HW * q + 4 * lane + c] = macc[q][c][m];
    }
    __syncthreads();
    gemv_sum_waves_store<MT, CWL * QPL, WAVES>(red, tid, cb, sk, S, N, ldy, bias, Y, part);
  } else {
    gemv_reduce_store<MT, CWL, WAVES>(acc, red, tid, cb, sk, S, N, ldy, bias, Y, part);
  }
}

// M <= 2 with the activations read directly (no LDS staging): the rows of a
// workgroup's k-range [rb, re) are dealt to its RL row-lanes in sweeps -- slot
// j of row-lane rl is packed row rb + j * RL + rl -- and a batch is BR
// consecutive slots.  So every batch is one contiguous run of BR * RL rows
// read by the whole workgroup at once, and the rows a lane processes first are
// the ones the memory system returns first: the dequant and dot products of
// the first slots overlap the arrival of the later ones instead of waiting
// for the lane's whole run.  Each slot has its own group, so its scale and
// zero loads are its own.  Slots past `re` load nothing (out-of-range offsets
// read zeros: a zero activation makes their products exactly zero), so every
// lane runs the same loads and the same trip count without a branch.
//
// The time to the first weight load is on the critical path of a few-us call
// (every wave waits for its own), so the set-up is kept short: the library is
// built to have the dispatch preload a kernel's leading arguments into SGPRs
// (-mllvm -amdgpu-kernarg-preload-count; fourteen SGPRs here), and the two
// entry points below order the arguments so that those SGPRs hold everything
// the first batch's loads need -- the first weight load then waits for no
// kernel-argument load at all, and the later arguments are loaded while the
// weights are in flight (measured on MI355X, C2: 4.69 -> 4.49 us against one
// batch of argument loads in front of everything).  Unsplit launches
// (gemv_direct_kernel) preload the operand pointers, N, K, the rows per
// workgroup, the grid size and the group reciprocal; split launches
// (gemv_direct_split_kernel) need the reciprocal of the column-block count
// too (block -> k-split, column block), and take X among the later
// arguments: its first load comes after the first slot's weight, scale and
// zero loads.  Each slot's loads are issued together, weight first (the long
// pole: cold HBM, most of the bytes).  Measured on MI355X, C2 (16 waves, two
// slots per lane, one batch), medians of 7 interleaved runs: 4.81-4.85 us
// with contiguous runs per lane, 4.68-4.70 with sweeps.
template <int MT, int CWL, int WAVES, bool ONE_BATCH, bool SPLIT, bool AZ>
__device__ __forceinline__ void gemv_direct_body(
    const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ X, int N, int K, int rows_per_wg,
    int nb, uint32_t gmagic, int gshift, uint32_t bmagic, int bshift, int ldx, int ldy,
    const f16* __restrict__ bias, f16* __restrict__ Y, float* __restrict__ part) {
  static_assert(MT <= 2, "direct activations are for M <= 2");
  constexpr int BR = GemvShape<WAVES>::kBatch;
  // 32-column and wider blocks: the CWL / 4 lane quads of a packed row each
  // load their row's activation octet once, one dword per lane, and rebuild
  // it with four quad-permute moves, instead of every lane loading all 16
  // bytes (12 fewer bytes through the load-return path per lane and slot, 4
  // more VALU).  Measured on MI355X, M = 1: K = 4096, N = 6144 6.80 -> 6.40
  // us; N = 8192 6.85 -> 6.56; K = 14336, N = 4096 11.74 -> 11.49.  On
  // 16-column blocks (C2) it measured slower (4.74 -> 4.79).
  constexpr bool kXShare = CWL >= 8;
  constexpr int RW = 64 / CWL;             // row-lanes per wave
  constexpr int RL = WAVES * RW;           // row-lanes per workgroup
  constexpr int CW = 4 * CWL;              // columns per workgroup
  __shared__ float red[WAVES][MT][CW];

  // XCD-aware block order (gemv_kernel), then block -> (k-split, column block)
  const int b0 = (int)blockIdx.x;
  const int lin = (nb & 7) == 0 ? (b0 & 7) * (nb >> 3) + (b0 >> 3) : b0;
  const int nblk = (N + CW - 1) / CW;
  // split launches (nb = nblk * splits): lin = sk * nblk + cb
  const int sk = SPLIT ? (int)((__umulhi((uint32_t)lin, bmagic) + (uint32_t)lin) >> bshift) : 0;
  const int cb = lin - sk * nblk;
  constexpr int S = SPLIT ? 2 : 1;   // the epilogue only asks whether the launch is split

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cq = lane % CWL;
  const int rl = wave * RW + lane / CWL;
  const int n = cb * CW + 4 * cq;
  const bool nv = n < N;
  const int KP = K >> 3;
  auto group_of = [&](int k) {
    return (int)((__umulhi((uint32_t)k, gmagic) + (uint32_t)k) >> gshift);
  };
  const int NG = group_of(K);
  const int rb = sk * rows_per_wg;
  const int re = min(KP, rb + rows_per_wg);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(MT - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);
  const uint32_t row_bytes = (uint32_t)N * 4u;
  // this lane's row and column at slot 0; slot j adds j * RL rows (in the SGPR)
  const uint32_t w_voff = ((uint32_t)(rb + rl) * (uint32_t)N + (uint32_t)n) * 4u;

  struct Batch {
    uint2 s[BR], z[BR];
    uint4 x[MT * BR];     // kXShare: the lane's dword in .x
    uint4 w[BR];
  };
  // Slots b * BR .. b * BR + BR - 1: offsets first, then the loads in the
  // order they are consumed, each slot's weight first.
  auto load_batch = [&](int b, Batch& bt) {
    uint32_t wo[BR], so[BR], xo[BR];
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      const int r = rb + (b * BR + i) * RL + rl;
      const bool v = nv && r < re;
      wo[i] = v ? w_voff : kOobOffset;
      so[i] = v ? ((uint32_t)group_of(r * 8) * (uint32_t)N + (uint32_t)n) * 2u : kOobOffset;
      // a shared octet is loaded whatever the lane's columns: its quad needs it
      xo[i] = kXShare ? (r < re ? (uint32_t)r * 16u + 4u * (uint32_t)(lane & 3) : kOobOffset)
                      : (v ? (uint32_t)r * 16u : kOobOffset);
    }
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      bt.w[i] = buf_load16<kNonTemporal>(rw, wo[i],
                                         uniform((uint32_t)((b * BR + i) * RL) * row_bytes));
      bt.s[i] = buf_load8(rs, so[i], 0u);
      bt.z[i] = buf_load8(rz, so[i], 0u);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if constexpr (kXShare)
          bt.x[m * BR + i].x = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
              rx, (int)xo[i], (int)uniform((uint32_t)m * (uint32_t)ldx * 2u), 0);
        else
          bt.x[m * BR + i] = buf_load16(rx, xo[i], uniform((uint32_t)m * (uint32_t)ldx * 2u));
      __builtin_amdgcn_sched_barrier(0);   // keep the slots in order
    }
  };

  Batch ba, bb;
  load_batch(0, ba);

  const MagicRegs mg = make_magic();
  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  auto process = [&](const Batch& bt) {
#pragma unroll
    for (int i = 0; i < BR; ++i) {
      const ColQ2 p01 = make_colq2<AZ>(bt.s[i].x, bt.z[i].x);
      const ColQ2 p23 = make_colq2<AZ>(bt.s[i].y, bt.z[i].y);
      const ColQ cq4[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
      f16x2 d[4][4];
      dq_word_fast<AZ>(bt.w[i].x, cq4[0], mg, d[0]);
      dq_word_fast<AZ>(bt.w[i].y, cq4[1], mg, d[1]);
      dq_word_fast<AZ>(bt.w[i].z, cq4[2], mg, d[2]);
      dq_word_fast<AZ>(bt.w[i].w, cq4[3], mg, d[3]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        uint4 xo4 = bt.x[m * BR + i];
        if constexpr (kXShare) {
          // quad_perm [k, k, k, k]: every lane of the quad takes lane k's dword
          const int xd = (int)xo4.x;
          xo4 = make_uint4((uint32_t)__builtin_amdgcn_update_dpp(0, xd, 0x00, 0xF, 0xF, false),
                           (uint32_t)__builtin_amdgcn_update_dpp(0, xd, 0x55, 0xF, 0xF, false),
                           (uint32_t)__builtin_amdgcn_update_dpp(0, xd, 0xAA, 0xF, 0xF, false),
                           (uint32_t)__builtin_amdgcn_update_dpp(0, xd, 0xFF, 0xF, 0xF, false));
        }
        const uint4 xp = perm_pairs(xo4);
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
  };

  // ONE_BATCH (the host's choice when every split has at most one batch, e.g.
  // C2): straight-line code, so the compiler's waits release slot 0 while the
  // later slots are still in flight (behind a branch shared with the loop it
  // waited for all of them).  Otherwise two register batches used ping-pong;
  // the batch count is the same for every lane, so the branches are uniform.
  if constexpr (ONE_BATCH) {
    process(ba);
  } else {
    const int nbat = (re - rb + BR * RL - 1) / (BR * RL);
    for (int b = 0; b < nbat; b += 2) {
      load_batch(b + 1, bb);
      process(ba);
      if (b + 1 >= nbat) break;
      load_batch(b + 2, ba);
      process(bb);
    }
  }

  gemv_reduce_store<MT, CWL, WAVES>(acc, red, tid, cb, sk, S, N, ldy, bias, Y, part);
}

// Unsplit launches: the first fourteen SGPRs of arguments (preloaded) are what
// the first batch's loads need.
template <int MT, int CWL, int WAVES, bool ONE_BATCH, bool AZ>
__global__ __launch_bounds__(64 * WAVES) void gemv_direct_kernel(
    const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ X, int N, int K, int rows_per_wg,
    int nb, uint32_t gmagic, int gshift, int ldx, int ldy, const f16* __restrict__ bias,
    f16* __restrict__ Y) {
  gemv_direct_body<MT, CWL, WAVES, ONE_BATCH, false, AZ>(QW, SC, ZR, X, N, K, rows_per_wg, nb,
                                                     gmagic, gshift, 0u, 0, ldx, ldy, bias, Y,
                                                     nullptr);
}

// Split launches: the block reciprocal joins the preloaded arguments, X
// follows them.
template <int MT, int CWL, int WAVES, bool ONE_BATCH, bool AZ>
__global__ __launch_bounds__(64 * WAVES) void gemv_direct_split_kernel(
    const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, int N, int K, int rows_per_wg, int nb, uint32_t bmagic,
    int bshift, uint32_t gmagic, int gshift, const f16* __restrict__ X, int ldx,
    float* __restrict__ part) {
  gemv_direct_body<MT, CWL, WAVES, ONE_BATCH, true, AZ>(QW, SC, ZR, X, N, K, rows_per_wg, nb,
                                                    gmagic, gshift, bmagic, bshift, ldx, 0,
                                                    nullptr, nullptr, part);
}

template <int MT, int CWL, int WAVES, bool STAGE, bool MF, int QPL, bool AZ>
hipError_t launch_cwlz(const GemmArgs& a, int split, void* ws, hipStream_t st) {
  constexpr int CW = 4 * CWL * QPL;
  const int nblk = (a.N + CW - 1) / CW;
  const int rows = gemv_rows_per_split(a.K, split);
  float* part = split > 1 ? static_cast<float*>(ws) : nullptr;
  const GroupDiv gd = group_div(a.G);
  if constexpr (MT <= 2 && !STAGE) {
    // every split's rows fit one batch of BR slots per row-lane
    constexpr int kRowsPerBatch = GemvShape<WAVES>::kBatch * WAVES * (64 / CWL);
    const bool one = rows <= kRowsPerBatch;
    const dim3 grid(nblk * split), block(GemvShape<WAVES>::kThreads);
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(a.qw);
    const uint16_t* sc = static_cast<const uint16_t*>(a.sc);
    const uint16_t* zr = static_cast<const uint16_t*>(a.zr);
    const f16* x = static_cast<const f16*>(a.x);
    if (split == 1) {
      auto kern = one ? gemv_direct_kernel<MT, CWL, WAVES, true, AZ>
                      : gemv_direct_kernel<MT, CWL, WAVES, false, AZ>;
      hipLaunchKernelGGL(kern, grid, block, 0, st, qw, sc, zr, x, a.N, a.K, rows, nblk, gd.magic,
                         gd.shift, a.ldx, a.ldy, static_cast<const f16*>(a.bias),
                         static_cast<f16*>(a.y));
    } else {
      auto kern = one ? gemv_direct_split_kernel<MT, CWL, WAVES, true, AZ>
                      : gemv_direct_split_kernel<MT, CWL, WAVES, false, AZ>;
      const GroupDiv bd = group_div(nblk);
      hipLaunchKernelGGL(kern, grid, block, 0, st, qw, sc, zr, a.N, a.K, rows, nblk * split,
                         bd.magic, bd.shift, gd.magic, gd.shift, x, a.ldx, part);
    }
  } else
    hipLaunchKernelGGL((gemv_kernel<MT, CWL, WAVES, STAGE, MF, QPL, AZ>), dim3(nblk * split),
                       dim3(GemvShape<WAVES>::kThreads), 0, st,
                       reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                       static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.x), a.N, a.K,
                       rows, split, gd.magic, gd.shift, a.ldx, a.ldy,
                       static_cast<const f16*>(a.bias), static_cast<f16*>(a.y), part);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || split == 1) return e;
  return launch_splitk_reduce(part, a.bias, a.y, a.M, a.N, a.ldy, split, st);
}

// Zero-point form by the call (w4a16_device.h): the kernels for integer zeros
// or those for any fp16 zero.
template <int MT, int CWL, int WAVES, bool STAGE, bool MF = false, int QPL = 1>
hipError_t launch_cwl(const GemmArgs& a, int split, void* ws, hipStream_t st) {
  return a.any_zeros ? launch_cwlz<MT, CWL, WAVES, STAGE, MF, QPL, true>(a, split, ws, st)
                     : launch_cwlz<MT, CWL, WAVES, STAGE, MF, QPL, false>(a, split, ws, st);
}

template <int MT, int WAVES, bool STAGE>
hipError_t launch_w(const GemmArgs& a, int cols, int split, void* ws, hipStream_t st) {
  switch (cols) {
    case 16: return launch_cwl<MT, 4, WAVES, STAGE>(a, split, ws, st);
    case 32: return launch_cwl<MT, 8, WAVES, STAGE>(a, split, ws, st);
    case 64: return launch_cwl<MT, 16, WAVES, STAGE>(a, split, ws, st);
    case 128: return launch_cwl<MT, 32, WAVES, STAGE>(a, split, ws, st);
    case 256: return launch_cwl<MT, 64, WAVES, STAGE>(a, split, ws, st);
    default: return hipErrorInvalidValue;
  }
}

// cfg 1 / 2: 8 / 16 waves; cfg 4 / 5: the same with the activations staged in
// LDS for M <= 2 (larger M always stages them); cfg 6 / 7: 16 / 8 waves,
// staged, with the dot products on the matrix cores (M <= 2, 64- or 128-column
// blocks only).  16 waves only for M <= 2 (the reduction buffer grows with waves x
// M).  cfg 0 / 3 (4 waves) measured slower everywhere and were retired.
template <int MT>
hipError_t launch_mt(const GemmArgs& a, int cols, int cfg, int split, void* ws, hipStream_t st) {
  if constexpr (MT <= 2) {
    switch (cfg) {
      case 1: return launch_w<MT, 8, false>(a, cols, split, ws, st);
      case 2: return launch_w<MT, 16, false>(a, cols, split, ws, st);
      case 4: return launch_w<MT, 8, true>(a, cols, split, ws, st);
      case 5: return launch_w<MT, 16, true>(a, cols, split, ws, st);
      case 6:
        if (cols == 64) return launch_cwl<MT, 16, 16, true, true, 1>(a, split, ws, st);
        if (cols == 128) return launch_cwl<MT, 16, 16, true, true, 2>(a, split, ws, st);
        return hipErrorInvalidValue;
      case 7:
        if (cols == 64) return launch_cwl<MT, 16, 8, true, true, 1>(a, split, ws, st);
        if (cols == 128) return launch_cwl<MT, 16, 8, true, true, 2>(a, split, ws, st);
        return hipErrorInvalidValue;
      default: return hipErrorInvalidValue;
    }
  } else {
    if (cfg != 1) return hipErrorInvalidValue;
    return launch_w<MT, 8, false>(a, cols, split, ws, st);
  }
}

}  // namespace

bool gemv_cols_valid(int cols) {
  return cols == 16 || cols == 32 || cols == 64 || cols == 128 || cols == 256;
}
bool gemv_cfg_valid(int cfg, int M, int cols) {
  return cfg == 1 || (M <= 2 && (cfg == 2 || cfg == 4 || cfg == 5)) ||
         (M <= 2 && (cols == 64 || cols == 128) && (cfg == 6 || cfg == 7));
}

int gemv_rows_per_split(int K, int split) {
  const int KP = K / 8;
  // whole 8-row batches per split keep every batch inside the batch alignment
  const int rows = (KP + split - 1) / split;
  return (rows + 7) / 8 * 8;
}

size_t gemv_workspace_bytes(int M, int N, int K, int split) {
  (void)K;
  if (split <= 1) return 0;
  return (size_t)split * (size_t)M * (size_t)N * sizeof(float);
}

hipError_t launch_gemv(const GemmArgs& a, int cols, int cfg, int split, void* ws, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_mt<1>(a, cols, cfg, split, ws, st);
    case 2: return launch_mt<2>(a, cols, cfg, split, ws, st);
    case 3: return launch_mt<3>(a, cols, cfg, split, ws, st);
    case 4: return launch_mt<4>(a, cols, cfg, split, ws, st);
    case 5: return launch_mt<5>(a, cols, cfg, split, ws, st);
    case 6: return launch_mt<6>(a, cols, cfg, split, ws, st);
    case 7: return launch_mt<7>(a, cols, cfg, split, ws, st);
    case 8: return launch_mt<8>(a, cols, cfg, split, ws, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
