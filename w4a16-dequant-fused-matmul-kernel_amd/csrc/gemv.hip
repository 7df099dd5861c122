// Decode GEMV for small M (M <= 8): Y = X @ dequant(qweight) streamed from HBM.
//
// Replaces the decode regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128 at M = 1..16, BLOCK_M >= 16).
//
// Layout of the work:
//   * a workgroup (WAVES waves) owns a block of CW = 4*CWL consecutive columns;
//     in a wave, CWL lanes cover one packed row (one dwordx4 = 4 columns per
//     lane) and the wave's 64/CWL row-lanes sit on different packed rows;
//   * each row-lane owns a contiguous run of packed rows, cut into batches of BR
//     rows (4 with 8 waves, 2 with 16 waves) aligned to absolute multiples of BR.
//     With G % 32 == 0 every 4-row half (32 k) lies in one quantisation group,
//     so a batch needs one scale/zero load per half;
//   * every load of batch i+1 is issued before batch i is consumed, in the order
//     scales, activations, weights, so the in-order vmcnt counter releases the
//     first weight row as soon as it lands.  Weights are read with the
//     non-temporal hint: each byte is used once;
//   * activations: for M <= 2 each lane reads its rows' activations directly
//     (the whole X is a few KiB and stays in L2), with no barrier before the
//     first weight arrives; for larger M, X is staged once per chunk in LDS,
//     permuted to the dequantiser's pair order;
//   * dequant is the packed-fp16 magic-number form (w4a16_device.h); the dot
//     product is v_dot2_f32_f16 with fp32 accumulation; no MFMA is used;
//   * reduction over row-lanes: a fixed xor-shuffle tree inside the wave, then the
//     waves in order through LDS -- deterministic;
//   * workgroup -> column block is XCD-aware: the hardware deals workgroups to the
//     8 XCDs round-robin, and consecutive column blocks are given to the same XCD
//     so that neighbouring row segments share that XCD's L2 lines;
//   * split-K where the column blocks cannot fill the CUs and K is long (the
//     planner's rule; a plan can also force it): each workgroup writes fp32
//     partials and a second kernel sums the splits in split order
//     (deterministic).
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

template <int MT, int CWL, int WAVES, bool STAGE>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(
    const f16* __restrict__ X, const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, const f16* __restrict__ bias, f16* __restrict__ Y,
    float* __restrict__ part, int N, int K, int ldx, int ldy, uint32_t gmagic, int gshift,
    int rows_per_wg, int S, int nblk) {
  constexpr int kThreads = GemvShape<WAVES>::kThreads;
  constexpr int BR = GemvShape<WAVES>::kBatch;
  constexpr int RH = BR < 4 ? BR : 4;      // rows per half (a half lies in one group)
  constexpr int H = BR / RH;               // halves per batch
  // activations read directly from global (M <= 2 unless STAGE) or staged in LDS
  constexpr bool XD = MT <= 2 && !STAGE;
  constexpr int RW = 64 / CWL;             // row-lanes per wave
  constexpr int RL = WAVES * RW;           // row-lanes per workgroup
  constexpr int CW = 4 * CWL;              // columns per workgroup
  constexpr int CHUNK = XD ? BR : kXsEntries / MT / BR * BR;   // packed rows of X per stage
  static_assert(CHUNK % BR == 0, "chunk must hold whole batches");
  __shared__ uint4 xs[XD ? 1 : MT * CHUNK];
  __shared__ float red[WAVES][MT][CW];

  // 16-column blocks: every kernel argument in one batch of scalar loads up
  // front (left to the compiler, the pointers are read only after the
  // block-order branches, a second and third dependent kernarg round trip
  // before the first weight load).  Measured on MI355X: C2 5.01 -> 4.86 us,
  // M = 2 5.50 -> 5.29 us, but K = 14336 N = 4096 12.96 -> 13.24 us; the
  // 32-column kernel measured 2-3 % slower with it, so it keeps the compiler's
  // order.
  const int nb = (int)gridDim.x;
  if constexpr (CWL <= 4)
    asm volatile("" ::"s"(X), "s"(QW), "s"(SC), "s"(ZR), "s"(bias), "s"(Y), "s"(part), "s"(N),
                 "s"(K), "s"(ldx), "s"(ldy), "s"(gmagic), "s"(gshift), "s"(rows_per_wg), "s"(S),
                 "s"(nblk), "s"(nb));

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
  const int n = cb * CW + 4 * cq;
  const bool nv = n < N;
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

  struct Batch {
    uint2 s[H], z[H];
    uint4 x[XD ? MT * BR : 1];
    uint4 w[BR];
  };
  // Rows r0..r0+BR-1 of this lane's run [.., le).  Row u rides in the SGPR
  // offset; weight rows at or past `le` (only in a run's last batch) read as zero.
  auto load_batch = [&](int r0, int le, Batch& b) {
#pragma unroll
    for (int h = 0; h < H; ++h) {
      // the group differs between row-lanes: its offset goes in the VGPR operand
      const int g = min(group_of((r0 + RH * h) * 8), NG - 1);
      // a batch past the lane's run (issued only to keep the loads the same
      // on every path) reads nothing from memory
      const uint32_t so = (nv && r0 < le) ? s_voff + (uint32_t)g * (uint32_t)N * 2u : kOobOffset;
      b.s[h] = buf_load8(rs, so, 0u);
      b.z[h] = buf_load8(rz, so, 0u);
    }
    if constexpr (XD) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int u = 0; u < BR; ++u)
          b.x[m * BR + u] = buf_load16(
              rx, r0 < le ? ((uint32_t)m * (uint32_t)ldx + (uint32_t)r0 * 8u) * 2u : kOobOffset,
              uniform((uint32_t)u * 16u));
    }
    // One path for full and partial batches (a lane-dependent branch here would
    // move the row offset out of the SGPR and serialise the loads).
    const uint32_t base = nv ? ((uint32_t)r0 * (uint32_t)N + (uint32_t)n) * 4u : kOobOffset;
#pragma unroll
    for (int u = 0; u < BR; ++u)
      b.w[u] = buf_load16<kNonTemporal>(rw, r0 + u < le ? base : kOobOffset,
                                        uniform((uint32_t)u * row_bytes));
  };

  auto process = [&](const Batch& b, int r0, int le, int c0) {
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const ColQ2 p01 = make_colq2(b.s[h].x, b.z[h].x), p23 = make_colq2(b.s[h].y, b.z[h].y);
      const ColQ cq4[4] = {colq_of<0>(p01), colq_of<1>(p01), colq_of<0>(p23), colq_of<1>(p23)};
#pragma unroll
      for (int uu = 0; uu < RH; ++uu) {
        const int u = h * RH + uu;
        const int r = r0 + u;
        if (r >= le) break;
        f16x2 d[4][4];
        dq_word_fast(b.w[u].x, cq4[0], mg, d[0]);
        dq_word_fast(b.w[u].y, cq4[1], mg, d[1]);
        dq_word_fast(b.w[u].z, cq4[2], mg, d[2]);
        dq_word_fast(b.w[u].w, cq4[3], mg, d[3]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          uint4 xp;
          if constexpr (XD)
            xp = perm_pairs(b.x[m * BR + u]);
          else
            xp = xs[m * CHUNK + (r - c0)];
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

  for (int c0 = rb; c0 < re; c0 += (XD ? re - rb : CHUNK)) {
    const int c1 = XD ? re : min(re, c0 + CHUNK);
    const int nr = c1 - c0;
    // this row-lane's rows in the chunk: BR-row aligned run
    const int per = ((nr + RL - 1) / RL + BR - 1) / BR * BR;
    const int lb = min(c1, c0 + rl * per);
    const int le = min(c1, lb + per);

    Batch ba, bb;
    if constexpr (XD) {
      load_batch(lb, le, ba);
    } else {
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
        if (idx < MT * CHUNK) xs[idx] = perm_pairs(xv[i]);
      }
      __syncthreads();
    }

    // Two register batches used ping-pong.  M <= 2: the trip count is the same
    // for every lane (`per` rows; past its own run a lane's loads read nothing
    // and process() skips its rows), and the loads are unconditional, so every
    // path has the same loads in flight and the compiler's waits count
    // exactly (with lane-dependent branches around the loads, its waits at the
    // joins covered the next batch too: 2-10 % slower on multi-batch runs); a
    // one-batch run (C2) has nothing to prefetch and skips the loop.  M > 2
    // keeps the per-lane loop, which measured 6-7 % faster there (M = 3, 4,
    // K = 4096, N = 28672).
    if constexpr (MT <= 2) {
      const int nbat = per / BR;
      if (nbat == 1) {
        process(ba, lb, le, c0);
      } else {
        for (int i = 0; i < nbat; i += 2) {
          const int r0 = lb + i * BR;
          load_batch(r0 + BR, le, bb);
          process(ba, r0, le, c0);
          load_batch(r0 + 2 * BR, le, ba);
          process(bb, r0 + BR, le, c0);
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

  // Reduce over row-lanes in a fixed order.  Inside each 16-lane DPP row the
  // lanes with equal cq are combined by row rotations, then a transpose-reduce
  // over the wave's four 16-lane rows leaves column slot c of the lane's quad in
  // row c (register-to-register, fixed order); the per-wave sums go through LDS
  // once and thread t < CW adds the WAVES partial sets of its column in wave
  // order.
  constexpr int PS = WAVES;   // partial sets per workgroup
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
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m)
      *reinterpret_cast<float4*>(&red[wave][m][4 * cq]) =
          make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
  }
  __syncthreads();

  const int t = tid;
  const int col = cb * CW + t;
  const bool cv = (t < CW) && (col < N);
  float v[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float s = 0.0f;
    if (t < CW) {
      s = red[0][m][t];
#pragma unroll
      for (int w = 1; w < PS; ++w) s += red[w][m][t];
    }
    v[m] = s;
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

template <int MT, int CWL, int WAVES, bool STAGE>
hipError_t launch_cwl(const GemmArgs& a, int split, void* ws, hipStream_t st) {
  constexpr int CW = 4 * CWL;
  const int nblk = (a.N + CW - 1) / CW;
  const int rows = gemv_rows_per_split(a.K, split);
  float* part = split > 1 ? static_cast<float*>(ws) : nullptr;
  const GroupDiv gd = group_div(a.G);
  hipLaunchKernelGGL((gemv_kernel<MT, CWL, WAVES, STAGE>), dim3(nblk * split),
                     dim3(GemvShape<WAVES>::kThreads), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const uint16_t*>(a.sc),
                     static_cast<const uint16_t*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), part, a.N, a.K, a.ldx, a.ldy, gd.magic, gd.shift, rows,
                     split, nblk);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || split == 1) return e;
  return launch_splitk_reduce(part, a.bias, a.y, a.M, a.N, a.ldy, split, st);
}

template <int MT, int WAVES, bool STAGE>
hipError_t launch_w(const GemmArgs& a, int cols, int split, void* ws, hipStream_t st) {
  switch (cols) {
    case 16: return launch_cwl<MT, 4, WAVES, STAGE>(a, split, ws, st);
    case 32: return launch_cwl<MT, 8, WAVES, STAGE>(a, split, ws, st);
    case 64: return launch_cwl<MT, 16, WAVES, STAGE>(a, split, ws, st);
    case 256: return launch_cwl<MT, 64, WAVES, STAGE>(a, split, ws, st);
    default: return hipErrorInvalidValue;
  }
}

// cfg 1 / 2: 8 / 16 waves; cfg 4 / 5: the same with the activations staged in
// LDS for M <= 2 (larger M always stages them).  16 waves only for M <= 2
// (the reduction buffer grows with waves x M).  cfg 0 / 3 (4 waves) measured
// slower everywhere and were retired.
template <int MT>
hipError_t launch_mt(const GemmArgs& a, int cols, int cfg, int split, void* ws, hipStream_t st) {
  if constexpr (MT <= 2) {
    switch (cfg) {
      case 1: return launch_w<MT, 8, false>(a, cols, split, ws, st);
      case 2: return launch_w<MT, 16, false>(a, cols, split, ws, st);
      case 4: return launch_w<MT, 8, true>(a, cols, split, ws, st);
      case 5: return launch_w<MT, 16, true>(a, cols, split, ws, st);
      default: return hipErrorInvalidValue;
    }
  } else {
    if (cfg != 1) return hipErrorInvalidValue;
    return launch_w<MT, 8, false>(a, cols, split, ws, st);
  }
}

}  // namespace

bool gemv_cols_valid(int cols) { return cols == 16 || cols == 32 || cols == 64 || cols == 256; }
bool gemv_cfg_valid(int cfg, int M) { return cfg == 1 || (M <= 2 && (cfg == 2 || cfg == 4 || cfg == 5)); }

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
