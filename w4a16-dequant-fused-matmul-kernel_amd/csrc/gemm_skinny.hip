// Skinny-M W4A16 GEMM (3 <= M <= 64 by the planner's choice; any M <= 64 by
// plan) on gfx950 matrix cores (v_mfma_f32_16x16x32_f16), weights streamed
// from HBM.
//
// Replaces the small-batch regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128 with BLOCK_M = 16..64).
//
// At these M the GEMM is still bound by the weight stream, and a prefill tiling
// (hundreds of rows per workgroup) leaves most CUs idle.  Here:
//   * a workgroup of 4, 8 or 16 waves owns a block of columns and the whole of
//     K, so no cross-workgroup reduction is needed.  Block widths (plan
//     tile_cfg):
//     - cfg 0: 16 columns, one per lane: one 4-byte weight load per lane and
//       32-k step, 2-byte scale / zero loads (N = 4096 gives 256 workgroups);
//     - cfg 2: 32 columns (M <= 32, N even), two adjacent columns per lane: one
//       8-byte weight load, 4-byte scale / zero loads, and the lane's
//       activation fragment feeds both n-tiles (X streamed once per 32
//       columns);
//     - cfg 3: 64 columns (M <= 16, N % 4 == 0), four columns per lane: one
//       16-byte weight load, 8-byte scale / zero loads;
//   * in v_mfma_f32_16x16x32_f16 lane l holds B[k = 8*(l/16)..+7][n = l%16]: one
//     packed int32 word.  A wave therefore covers 16 columns x 32 k per MFMA
//     and n-tile, reading 4 packed rows of its block per load;
//   * the waves split K into whole batches of 8 k-steps (256 k).  Up to
//     K = 4096 there are enough waves (K / 256, at least 4) for one batch
//     each, and each wave issues all its loads before its first product;
//     longer K deals the batches to 4 waves in sweeps (batch i of every wave
//     together is one contiguous run of K), each wave with two register
//     batches used ping-pong, all loads of batch i+1 -- weights, scales, zeros
//     and activations -- issued before batch i is consumed, unconditionally
//     (past the range they read zeros), so the compiler's wait counts are
//     exact;
//   * activations (MT x 16 rows) are read directly from global memory: the whole
//     X is a few hundred KiB and stays in L1/L2; rows past M read as zero through
//     the buffer range check.  On a 16-row tile with one batch per wave and
//     M >= 9 (XS) they come instead through the wave's own LDS slots, loaded
//     as whole rows (whole 128-byte lines) by LDS-direct loads;
//   * dequant is the packed-fp16 magic-number form; its pairs come out in the
//     order (w0 w4, w1 w5, w2 w6, w3 w7), and the MFMA's k order is matched by
//     permuting the activation fragment (one m-tile, or more n-tiles than
//     m-tiles) or else the words back to natural order;
//   * the waves' 16x16 fp32 tiles are summed in LDS in wave order
//     (deterministic) and rounded to fp16 once; optional fp16 bias add;
//   * workgroup -> column block is XCD-aware (consecutive blocks share an XCD).
// Requirements (checked by the caller): G % 32 == 0, K % G == 0, 16-byte
// aligned x, qweight aligned to the weight load (4 / 8 / 16 bytes for cfg
// 0 / 2 / 3) and scales / zeros to theirs (2 / 4 / 8 bytes), and x, qweight,
// scales, zeros each below 2 GiB.  Any N (cfg 2: even, cfg 3: N % 4 == 0).
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kBatch = 8;  // k-steps (32 k each) per batch

// GSTEP = k-steps per quantisation group inside an aligned 8-step batch (G/32
// when that is 1, 2, 4 or 8; 8 for larger powers of two): scales and zeros are
// loaded once per group.  GSTEP = 1 loads them every k-step (any G % 32 == 0).
// NT = columns per lane: 1 (16-column blocks) or 2 (32-column blocks, N even:
// the lane's two adjacent columns come in one 8-byte word load and one 4-byte
// scale / zero load each, and its activation fragment feeds both n-tiles, so a
// CU streams X once for 32 columns instead of once per 16).
//
// Arguments: the first fourteen SGPRs' worth are what the first loads need
// (operand pointers, M, N, K, the group reciprocal, the row groups, ldx); the
// library is built to have the dispatch preload them into SGPRs (-mllvm
// -amdgpu-kernarg-preload-count), so the first loads wait for no
// kernel-argument load, and the epilogue's arguments are loaded meanwhile.
// geo = row groups per column block | rows per group << 8 | group shift << 16;
// k / G is (umulhi(k, gmagic) + k) >> shift (group_div), no division; the
// grid size is nblk * mgs (no read of the dispatch packet).
template <int MT, int GSTEP, int WAVES, int NT, bool ONE_BATCH, bool AZ, bool XS>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(
    const f16* __restrict__ X, const uint32_t* __restrict__ QW, const uint16_t* __restrict__ SC,
    const uint16_t* __restrict__ ZR, int M, int N, int K, uint32_t gmagic, uint32_t geo, int ldx,
    int ldy, const f16* __restrict__ bias, f16* __restrict__ Y) {
  static_assert(NT == 1 || NT == 2 || NT == 4, "one, two or four columns per lane");
  static_assert(!XS || (ONE_BATCH && MT * NT <= 8), "staged activations: one batch per wave");
  constexpr int kWaves = WAVES;
  // XS: per wave and m-tile, 512 16-byte slots for the batch's activations
  // (16 rows x 512 B); once the wave's products are done the same space holds
  // its partial tiles.  Otherwise only the partial tiles, in red.  (Staged in
  // the 4-wave two-batch loop as well, with a second array for the other
  // register batch, it measured slower on MI355X: K = 11008 / 14336, N =
  // 4096, M = 32 17.4 / 21.5 -> 19.0 / 22.5 us, K = N = 5120, M = 24 12.8 ->
  // 14.0; one wave per SIMD does not hide the LDS round trip.)
  __shared__ uint4 xs[XS ? kWaves * MT * 512 : 1];
  __shared__ f32x4 red[XS ? 1 : kWaves][MT][NT][64];

  const int mgs = (int)(geo & 0xFFu), rpg = (int)((geo >> 8) & 0xFFu);
  const int gshift = (int)(geo >> 16);
  auto group_of = [&](uint32_t k) { return div_group(k, gmagic, gshift); };
  const int nb = (N + 16 * NT - 1) / (16 * NT) * mgs;
  int lin = (int)blockIdx.x;
  if ((nb & 7) == 0) lin = (lin & 7) * (nb >> 3) + (lin >> 3);
  // The workgroup owns rows [row0, row0 + rpg) of its column block: all of
  // them (mgs = 1, rpg = 16 MT) or one of mgs row groups of 16 or 8 rows
  // (MT = 1; tile rows past rpg load and store nothing), the groups of a
  // block on consecutive workgroups (one XCD, sharing its weights in L2).
  const int cb = mgs == 1 ? lin : lin / mgs;
  const int row0 = (lin - cb * mgs) * rpg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;       // column (pair for NT = 2) within the block
  const int q = lane >> 4;       // octet within a 32-k step
  const int col = cb * (16 * NT) + NT * c;   // the lane's first column
  const bool nv = col < N;                   // (N even for NT = 2: so is col + 1)
  const int KP = K >> 3;
  const int KS = K >> 5;         // 32-k steps
  const int NG = (int)group_of((uint32_t)K);

  const MagicRegs mg = make_magic();
  // partial tile (mt, t) of wave w, lane `lane`
  auto red_at = [&](int w, int mt, int t) -> f32x4& {
    if constexpr (XS)
      return reinterpret_cast<f32x4*>(xs)[w * MT * 512 + (mt * NT + t) * 64 + lane];
    else
      return red[w][mt][t][lane];
  };
  // rows of X lie ldx elements apart; the range ends after row M - 1's K
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(M - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(SC, (uint32_t)NG * (uint32_t)N * 2u);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZR, (uint32_t)NG * (uint32_t)N * 2u);

  // This wave's k-steps, in whole 8-step batches.  One batch per wave: a contiguous run of `per` steps.  The two-batch loop
  // deals the batches to the waves in sweeps instead: batch i of wave w is
  // steps (i W + w) 8 .. + 8, so batch i of every wave together is one
  // contiguous run of K, read by the workgroup at once (measured on MI355X
  // against a contiguous run per wave, cold weights, same run, µs: K = 14336,
  // N = 4096, M = 16 17.4 -> 17.2, 64-column blocks 26.2 -> 25.3; K = 8192,
  // N = 8192, M = 16, G = 32 18.7 -> 17.4; K = 13824, N = 5120, M = 8 17.2 ->
  // 16.8; planned plans -6.5 .. +0.4 %).  Either way batch starts are
  // multiples of 8 k-steps (256 k), so group boundaries fall on fixed slots.
  const int per = ((KS + kWaves - 1) / kWaves + kBatch - 1) / kBatch * kBatch;
  const int kb = ONE_BATCH ? min(KS, wave * per) : wave * kBatch;
  const int ke = ONE_BATCH ? min(KS, kb + per) : KS;
  const int bstep = ONE_BATCH ? kBatch : kWaves * kBatch;   // steps between a wave's batches

  // per-lane offsets at k = 0
  const uint32_t w_off = nv ? ((uint32_t)q * (uint32_t)N + (uint32_t)col) * 4u : kOobOffset;
  const uint32_t s_off = nv ? (uint32_t)col * 2u : kOobOffset;
  uint32_t x_off[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = row0 + mt * 16 + c;
    x_off[mt] = row < M && mt * 16 + c < rpg
                    ? ((uint32_t)row * (uint32_t)ldx + (uint32_t)q * 8u) * 2u
                    : kOobOffset;
  }

  // XS: load j of m-tile mt brings rows 2j and 2j + 1 of the tile (lanes 0-31
  // and 32-63), 16 B per lane of the batch's 512 B per row, so each load reads
  // eight whole 128-byte lines (the direct fragment loads read 16 rows x 64 B,
  // half of 16 lines each: measured on MI355X with same-byte loads, M = 16 /
  // 24 / 32, K = N = 4096, 6.68 / 7.85 / 7.95 -> 6.11 / 6.31 / 6.66 us).
  // Lane L writes slot 64 j + L, which holds chunk (L % 32) ^ (row % 16) of
  // its row, so a fragment read (16 rows, one chunk each) hits 16 distinct
  // 16-byte bank groups: the row r = 2j + L / 32 chunk (L % 32) ^ r sits at
  // slot 32 r + ((chunk) ^ r).
  // Chunks at or past the wave's last k-step (K % 256 != 0, or a wave with
  // fewer steps) and rows past M or past the row group read zero, as the
  // direct loads' past steps do (the past steps run branch-free against zero
  // weights, and a row's bytes past K may hold anything).  Never both offsets
  // out of range at once: their sum would wrap.
  const uint32_t xs_h = (uint32_t)(lane >> 5);
  const uint32_t xs_voff = xs_h * (uint32_t)ldx * 2u;
  const uint32_t xs_chunk = ((uint32_t)(lane & 31) ^ xs_h) << 4;   // load j: ^ (j << 5)
  const uint32_t xs_step = ((uint32_t)(lane & 31) ^ xs_h) >> 2;     // load j: ^ (j >> 1)
  uint4* const xs_wave = XS ? xs + wave * MT * 512 : xs;

  struct Batch {
    uint32_t w[kBatch][NT];
    uint32_t sz[kBatch][NT];  // scale bits | zero bits << 16
    uint4 x[kBatch][MT];
  };
  auto load_batch = [&](int s0, Batch& b) {
    if constexpr (XS) {
      // the activations first: loads retire in issue order, so the wait for
      // them before the first LDS read does not wait for the weights
      const uint32_t lim = (uint32_t)max(0, ke - s0);   // steps of the batch in range
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int r = mt * 16 + 2 * j;
          const bool rows_in = r < rpg && row0 + r < M;        // wave-uniform
          const uint32_t xo =
              uniform(rows_in ? (uint32_t)(row0 + r) * (uint32_t)ldx * 2u + (uint32_t)s0 * 64u : 0u);
          const uint32_t vo = rows_in && (xs_step ^ (uint32_t)(j >> 1)) < lim
                                  ? xs_voff + (xs_chunk ^ ((uint32_t)j << 5))
                                  : kOobOffset;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rx, (lds_void*)(xs_wave + mt * 512 + 64 * j), 16, vo, xo, 0, 0);
        }
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int ks = s0 + j;
      // every step issues its loads; steps past this wave's range (wave-uniform)
      // read zeros through an out-of-range offset and are never processed
      const bool in = ks < ke;
      {
        const uint32_t wk = uniform(in ? (uint32_t)ks * 4u * (uint32_t)N * 4u : kOobOffset);
        if constexpr (NT == 1) {
          b.w[j][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, (int)w_off, (int)wk, 0);
        } else if constexpr (NT == 2) {
          const uint2 w2 = buf_load8(rw, w_off, wk);
          b.w[j][0] = w2.x;
          b.w[j][1] = w2.y;
        } else {
          const uint4 w4 = buf_load16(rw, w_off, wk);
          b.w[j][0] = w4.x;
          b.w[j][1] = w4.y;
          b.w[j][2] = w4.z;
          b.w[j][3] = w4.w;
        }
        if (j % GSTEP == 0) {
          const uint32_t gk =
              uniform(in ? group_of((uint32_t)(ks * 32)) * (uint32_t)N * 2u : kOobOffset);
          if constexpr (NT == 1) {
            const uint32_t sv =
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)s_off, (int)gk, 0);
            const uint32_t zv =
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rz, (int)s_off, (int)gk, 0);
            b.sz[j][0] = (sv & 0xFFFFu) | (zv << 16);
          } else if constexpr (NT == 2) {
            const uint32_t sv =
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)s_off, (int)gk, 0);
            const uint32_t zv =
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rz, (int)s_off, (int)gk, 0);
            b.sz[j][0] = (sv & 0xFFFFu) | (zv << 16);
            b.sz[j][1] = (sv >> 16) | (zv & 0xFFFF0000u);
          } else {
            const uint2 sv = buf_load8(rs, s_off, gk);
            const uint2 zv = buf_load8(rz, s_off, gk);
            b.sz[j][0] = (sv.x & 0xFFFFu) | (zv.x << 16);
            b.sz[j][1] = (sv.x >> 16) | (zv.x & 0xFFFF0000u);
            b.sz[j][2] = (sv.y & 0xFFFFu) | (zv.y << 16);
            b.sz[j][3] = (sv.y >> 16) | (zv.y & 0xFFFF0000u);
          }
        } else {
#pragma unroll
          for (int t = 0; t < NT; ++t)   // same group as the batch slot it copies
            b.sz[j][t] = b.sz[j - j % GSTEP][t];
        }
        if constexpr (!XS) {
          const uint32_t xk = uniform(in ? (uint32_t)ks * 64u : kOobOffset);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) b.x[j][mt] = buf_load16(rx, x_off[mt], xk);
        }
      }
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{};

  auto process = [&](const Batch& b, int s0) {
    // XS: the batch's fragments, all read before the first product (one LDS
    // round trip per batch instead of one per step)
    uint4 xf[XS ? kBatch : 1][MT];
    if constexpr (XS) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xf[j][mt] = xs_wave[mt * 512 + 32 * c + ((4 * j + q) ^ c)];
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      // Steps past the range loaded zero activations and zero scales / zeros
      // (ke is a multiple of the group's step count, so a past step's group
      // slot is past too): their products are exactly 0.  Single-batch code
      // runs them branch-free: behind per-step range branches the compiler
      // sank the later steps' loads below the earlier steps' math, a round
      // trip each.  The two-batch loop skips them (measured faster there: C5
      // M = 16, K = 28672 took 47.4 us branch-free against 40.4).
      if (!ONE_BATCH && s0 + j >= ke) break;   // wave-uniform
      // Dequantised words come out in pair order (w0 w4, w1 w5, ...).  The
      // MFMA sums over k in whatever order both operands share, so either the
      // activation fragments (4 v_perm per m-tile) or the words (4 per word
      // and n-tile) are permuted, whichever is fewer: measured on MI355X,
      // 64-column blocks M = 1 / 4 / 16, K = 4096, N = 28672: 17.7 / 18.8 /
      // 21.2 -> 16.5 / 17.3 / 20.8 us with the activations permuted; M = 32 on
      // 32-column blocks (two m-tiles, two n-tiles) 11.9 vs 12.3 us the other way.
      constexpr bool kXPerm = MT == 1 || NT > MT;
      uint4 xa[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // XS: row c, chunk 4 j + q of the staged batch
        const uint4 xv = XS ? xf[j][mt] : b.x[j][mt];
        xa[mt] = kXPerm ? perm_pairs(xv) : xv;
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const ColQ cq = make_colq<AZ>(b.sz[j][t] & 0xFFFFu, b.sz[j][t] >> 16);
        f16x2 d[4];
        dq_word_fast<AZ>(b.w[j][t], cq, mg, d);
        // kXPerm: the words in pair order (w0 w4 w1 w5 w2 w6 w3 w7), the
        // activations permuted to match; else natural k order:
        // w0..w7 = d0.x d1.x d2.x d3.x d0.y d1.y d2.y d3.y
        const f16x8 bf = kXPerm ? f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y}
                                : f16x8{d[0].x, d[1].x, d[2].x, d[3].x, d[0].y, d[1].y, d[2].y, d[3].y};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(f16x8, xa[mt]), bf, acc[mt][t], 0, 0, 0);
      }
    }
  };

  // Two register batches used ping-pong.  The loads are unconditional and the
  // only branches (skipping a batch past the range, and the step check inside
  // process) contain no loads, so every path has the same loads in flight and
  // the compiler's vmcnt waits count exactly; with loads under the branches
  // its waits at the joins covered the next batch too (C3 M = 4..32 measured
  // 2-11 % slower that way).
  if constexpr (ONE_BATCH) {
    // Every load of the batch goes out before the first product: left to
    // itself the compiler (well under the register cap) sank the second
    // m-tile's activation loads below the first waits, a round trip each
    // (M = 24 / 32, K = N = 4096: 9.96 / 11.45 -> 9.64 / 10.95 us; 64-column
    // blocks M = 4..16 6-7 % faster).  Not with 3-4 m-tiles on 16 waves,
    // where holding every load spills (M = 64: 17.6 -> 23.4 us).
    Batch b1;
    load_batch(kb, b1);
    if constexpr (MT <= 2 || WAVES < 16) __builtin_amdgcn_sched_barrier(0);
    process(b1, kb);
  } else {
    Batch bt[2];
    load_batch(kb, bt[0]);
    for (int s0 = kb; s0 < ke; s0 += 2 * bstep) {
      load_batch(s0 + bstep, bt[1]);
      process(bt[0], s0);
      load_batch(s0 + 2 * bstep, bt[0]);
      if (s0 + bstep < ke) process(bt[1], s0 + bstep);
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) red_at(wave, mt, t) = acc[mt][t];
  __syncthreads();
  // wave w finishes tiles w, w + WAVES, ...: sum the waves in order, round, store
  for (int i = wave; i < MT * NT; i += kWaves) {
    const int mt = i / NT;
    {
      const int t = i % NT;
      f32x4 v = red_at(0, mt, t);
#pragma unroll
      for (int w = 1; w < kWaves; ++w) v += red_at(w, mt, t);
      if (nv) {
        const f16 bv = bias ? bias[col + t] : (f16)0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + mt * 16 + 4 * q + r;
          if (row < M && mt * 16 + 4 * q + r < rpg) {
            f16 y = f32_to_f16(v[r]);
            if (bias) y = y + bv;
            Y[(size_t)row * ldy + col + t] = y;
          }
        }
      }
    }
  }
}

// Waves per workgroup: as many as give each wave exactly one batch (K <= 1024:
// 4, K <= 2048: 8, K <= 4096: 16), so every load is issued before the first
// product, in one round trip to memory; longer K runs 4 waves in the
// two-batch loop (16 waves' loop registers spill; 8 or 16 waves in the loop
// measured no faster at K = 8192..28672).  Measured on MI355X, cold weights,
// against 4 waves in the loop: K = N = 4096 M = 4 / 8 / 16: 6.40 / 6.78 /
// 7.85 us -> 5.74 / 6.29 / 7.49; M = 16, N = 28672 (64 columns): 22.6 ->
// 21.1; M = 8, K = 2048, N = 4096: 4.99 -> 4.55 with 8 waves.
template <int MT, int GSTEP, int NT, bool AZ>
hipError_t launch_ntz(const GemmArgs& a, int rpg, hipStream_t st) {
  const int mgs = (a.M + rpg - 1) / rpg;
  const int nblk = (a.N + 16 * NT - 1) / (16 * NT);
  const int ks = a.K >> 5;
  // 16 waves hold 128 registers each: 64 rows with a scale / zero load per
  // step would spill there, and take the loop instead
  constexpr int k16 = MT == 4 && GSTEP == 1 ? 0 : 16;
  // Activations staged in LDS by whole-line loads (XS) on one 16-row tile
  // of 8 or 16 waves (64 / 128 KiB of LDS) that holds at least 9 rows: M >= 9
  // and 16-row groups or the whole tile.  Measured on MI355X against the direct fragment loads
  // (µs, G = 128, cold weights): K = N = 4096, M = 24 / 32 7.81 / 7.93 ->
  // 6.60 / 6.77; N = 6144, M = 16 / 32 (64-column blocks) 8.05 / 9.64 ->
  // 7.13 / 8.89; N = 14336 / 28672, M = 16 10.84 / 21.11 -> 10.06 / 19.74;
  // K = 2048, N = 4096, M = 32 5.28 -> 4.81; M = 9 / 12 / 15 on the whole
  // 16-row tile, K = 4096, N = 6144: 6.90 / 7.41 / 7.86 -> 6.65 / 6.83 / 7.06
  // (G = 32: 7.72 / 8.38 / 9.17 -> 7.06 / 7.26 / 7.58).  Not taken: M = 4
  // (1.6-4.4 % slower: a few rows gain nothing from whole lines and pay the
  // LDS round trip), M = 8 and 8-row groups (-7 .. +2 %), 4 waves (K <= 1024:
  // M = 16 8 % slower, M = 32 a tie).
  const bool xs = MT == 1 && rpg >= 16 && a.M >= 9;
  using Kernel = decltype(&skinny_kernel<MT, GSTEP, 4, NT, true, AZ, false>);
  constexpr int w16 = k16 ? k16 : 4;
  const Kernel k =
      ks <= 4 * kBatch     ? skinny_kernel<MT, GSTEP, 4, NT, true, AZ, false>
      : ks <= 8 * kBatch   ? (xs ? skinny_kernel<MT, GSTEP, 8, NT, true, AZ, MT == 1>
                                 : skinny_kernel<MT, GSTEP, 8, NT, true, AZ, false>)
      : ks <= k16 * kBatch ? (xs ? skinny_kernel<MT, GSTEP, w16, NT, true, AZ, MT == 1 && w16 == 16>
                                 : skinny_kernel<MT, GSTEP, w16, NT, true, AZ, false>)
                           : skinny_kernel<MT, GSTEP, 4, NT, false, AZ, false>;
  const int waves = ks <= 4 * kBatch ? 4 : ks <= 8 * kBatch ? 8 : ks <= k16 * kBatch ? k16 : 4;
  const GroupDiv gd = group_div(a.G);
  const uint32_t geo = (uint32_t)mgs | ((uint32_t)rpg << 8) | ((uint32_t)gd.shift << 16);
  hipLaunchKernelGGL(k, dim3(nblk * mgs), dim3(64 * waves), 0, st,
                     static_cast<const f16*>(a.x), reinterpret_cast<const uint32_t*>(a.qw),
                     static_cast<const uint16_t*>(a.sc), static_cast<const uint16_t*>(a.zr), a.M,
                     a.N, a.K, gd.magic, geo, a.ldx, a.ldy, static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y));
  return hipGetLastError();
}

// Zero-point form by the call (w4a16_device.h): the kernels for integer zeros
// or those for any fp16 zero.
template <int MT, int GSTEP, int NT>
hipError_t launch_nt(const GemmArgs& a, int rpg, hipStream_t st) {
  return a.any_zeros ? launch_ntz<MT, GSTEP, NT, true>(a, rpg, st)
                     : launch_ntz<MT, GSTEP, NT, false>(a, rpg, st);
}

template <int MT, int GSTEP>
hipError_t launch_g(const GemmArgs& a, int cfg, int rpg, hipStream_t st) {
  if constexpr (MT <= 2) {
    if (cfg == 2) return launch_nt<MT, GSTEP, 2>(a, rpg, st);   // 32-column blocks
  }
  if constexpr (MT == 1) {
    if (cfg == 3) return launch_nt<MT, GSTEP, 4>(a, rpg, st);   // 64-column blocks
  }
  return launch_nt<MT, GSTEP, 1>(a, rpg, st);                    // 16-column blocks
}

template <int MT>
hipError_t launch_mt(const GemmArgs& a, int cfg, int rpg, hipStream_t st) {
  // batch slots per group when group boundaries land on fixed slots of an
  // aligned 8-step (256-k) batch: G / 32 a power of two
  const int gs = a.G / 32;
  if (gs >= 8 && (gs & (gs - 1)) == 0) return launch_g<MT, 8>(a, cfg, rpg, st);
  switch (gs) {
    case 4: return launch_g<MT, 4>(a, cfg, rpg, st);
    case 2: return launch_g<MT, 2>(a, cfg, rpg, st);
    default: return launch_g<MT, 1>(a, cfg, rpg, st);
  }
}

}  // namespace

// cfg 0: 16-column blocks; 2: 32-column blocks (N even); 3: 64-column blocks
// (N % 4 == 0); the wave count follows K (launch_nt).  `rows`: rows of y per
// workgroup, all of them (M rounded up to 16) or 16, one row group per
// workgroup and M / 16 workgroups per column block, or 8 (half a tile, the
// other half's lanes load and store nothing): each workgroup then streams
// 16 (8) rows of X instead of all M (X's bytes per CU, not the weights',
// bound the kernel from M = 16 at K = N = 4096) and the weights are read once
// per row group, from L2 after the first.  32-column blocks hold at most two
// row tiles per workgroup, 64-column blocks one.  cfg 1 (8 waves in the
// two-batch loop on 16-column blocks) measured slower on every shape and was
// retired.
bool skinny_plan_valid(int cfg, int M, int N, int rows) {
  const int whole = (M + 15) / 16 * 16;
  if (M < 1 || M > kSkinnyMaxM || !(rows == whole || rows == 16 || rows == 8)) return false;
  if (cfg == 0) return true;
  if (cfg == 2) return rows <= 32 && N % 2 == 0;
  if (cfg == 3) return rows <= 16 && N % 4 == 0;
  return false;
}

hipError_t launch_skinny(const GemmArgs& a, int cfg, int rows, hipStream_t st) {
  if (!skinny_plan_valid(cfg, a.M, a.N, rows)) return hipErrorInvalidValue;
  switch (rows) {
    case 8:
    case 16: return launch_mt<1>(a, cfg, rows, st);
    case 32: return launch_mt<2>(a, cfg, rows, st);
    case 48: return launch_mt<3>(a, cfg, rows, st);
    case 64: return launch_mt<4>(a, cfg, rows, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
