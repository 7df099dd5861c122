// Prefill W4A16 GEMM on gfx950 matrix cores with activations and packed
// weights streamed into LDS by the buffer loads' LDS-direct form, and the
// weight dequant software-pipelined under the MFMAs
// (v_mfma_f32_16x16x32_f16, fp32 accumulation, two waves per SIMD).
//
// Replaces the large-M regime of the reference's fused kernel
// (w4a16-kernel/src/w4a16/triton_kernel.py:62-128: fp16 dequant of the weight
// tile, tl.dot with fp32 accumulation, fp16 store).
//
// Design:
//   * a workgroup of 4 waves owns a 128 x 256 tile of Y; each wave 128 rows x
//     64 columns = 8 x 4 tiles of 16 x 16, 128 accumulator registers, two waves
//     per SIMD;
//   * a lane's B operand for one 32-k half-step is one packed int32 word (8 k of
//     one column); columns are interleaved by 4 so one 16-byte word quad feeds
//     the wave's four n-tiles.  Words are dequantised in natural k order
//     (one v_perm_b32 per pair puts nibbles 2i and 2i+1 under the two fp16
//     magic numbers), so the activations need no permutation;
//   * activations: buffer_load_dwordx4 ... lds writes each 16-byte octet of the
//     workgroup's 128 x 64 slice straight into LDS, no VGPRs involved; rows are
//     128 bytes with the octet slot XOR-swizzled by (row / 2) % 8, so the
//     16-lane fragment reads hit 16 distinct 16-byte bank groups.  Two buffers;
//     step kt+1's slice is requested at the start of step kt and each wave
//     waits for its own part before the step's closing barrier;
//   * weights, scales and zeros: per wave, four LDS stages filled by
//     LDS-direct loads three steps ahead (each wave streams and reads back only
//     its own columns: no barrier); each stage is its own LDS array, so the
//     compiler's vmcnt wait before a stage's reads covers exactly the loads into
//     that stage.  One load per half-step (per step when G % 64 == 0: both
//     halves then share a group) brings the scales and zeros of the
//     wave's 64 columns, laid out per 4-column quad as (scales 0-1, scales 2-3,
//     zeros 0-1, zeros 2-3), so a lane reads its column constants with one
//     ds_read_b128; the load addresses both tensors through one buffer
//     resource based at the lower of the two (the launcher checks they lie
//     within 2 GiB of each other);
//   * loads retire in issue order: each step requests the next activation
//     slice before the weights three steps ahead, so the wait for activations
//     never waits for weights issued less than two steps back;
//   * software pipeline: a half-step's 32 MFMAs run beside the dequant of the
//     next half-step (inputs read from LDS one half-step earlier still), each
//     MFMA followed by two VALU instructions (sched_group_barrier): the matrix
//     core and the vector ALU work at the same time;
//   * every step issues the same loads (steps past the range read zeros
//     through an out-of-range offset) and the k-loop runs in whole blocks of
//     four steps, so no branch joins paths with different loads in flight (the
//     compiler's wait counts would fall back to vmcnt(0) there);
//   * XCD-aware grouped tile order, optional split-K (fp32 partials), fp16 RNE
//     epilogue with the optional fp16 bias add of W4A16Linear (linear.py:90-91).
// Requirements (checked by the caller): K % 256 == 0, split ranges of whole
// 4-step blocks (launch_wg), N % 4 == 0, G % 32 == 0, K % G == 0, 16-byte
// aligned x/qweight, 8-byte aligned scales/zeros/y/bias, and x, qweight,
// scales, zeros each below 2 GiB.
#include "w4a16_device.h"
#include "w4a16_launch.h"

#include <type_traits>

namespace w4a16 {
namespace {

constexpr int kBK = 64;
constexpr int kGroupM = 4;     // M-tiles per group of the tile order
constexpr int kNTiles = 4;     // 16-column MFMA tiles per wave (64 columns)
constexpr int kStages = 4;     // weight stages per wave (steps in flight)
constexpr int kWaves = 4;      // waves per workgroup, all along N
constexpr int kNT = 64 * kWaves;
constexpr int kBN = 16 * kNTiles * kWaves; // 256 columns
// kMT = 16-row MFMA tiles per wave: 8 (128-row workgroup tiles, prefill), 4
// or 2 (64 / 32 rows: small M, where a 128-row tile would spend most of its
// matrix-core time on rows past M; the dequant per weight is the same)

// Workgroup barrier for the activation tile: this wave's LDS accesses
// complete, then s_barrier.  __syncthreads() would also wait for every
// outstanding LDS-direct load (its fence covers all LDS writes, vmcnt(0)),
// draining the weight pipeline at every k-step.  The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Per column: zz = (1024 + zero, 64 + zero) as (low, high) halves, s = scale
// (AZ: zz = (zero, zero)).
struct ColN {
  f16x2 zz;
  f16 s;
};

// One packed word -> its 8 weights in natural order: d[i] = (w_2i, w_2i+1).
// v_perm_b32 copies byte i (nibbles 2i, 2i+1) into bytes 0 and 2; the mask
// keeps nibble 2i in bits [0,4) and nibble 2i+1 in bits [20,24), which the
// magic word 0x54006400 turns into the fp16 pair (1024 + q_2i, 64 + q_2i+1).
// Subtracting zz is exact for integer zero-points with |z| <= 1024, so the
// result is fp16(q - z) * s with one RNE rounding, as in the reference.  AZ
// (any fp16 zero): the magic word, which is also the fp16 pair (1024, 64), is
// subtracted first (exact: the codes), then the zero with the reference's
// rounding of fp16(q) - z.
template <bool AZ>
__device__ __forceinline__ void dq_word_nat(uint32_t w, const ColN& c, uint32_t magic_mix,
                                            f16x2 d[4]) {
  const f16x2 s2 = f16x2{c.s, c.s};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = __builtin_amdgcn_perm(w, w, 0x01010101u * (uint32_t)i);
    const f16x2 p = as_h2(and_or(t, 0x00F0000Fu, magic_mix));
    if constexpr (AZ)
      d[i] = ((p - as_h2(magic_mix)) - c.zz) * s2;
    else
      d[i] = (p - c.zz) * s2;
  }
}

// kSZ1: G % 64 == 0, so both half-steps of a step lie in one group and one
// scale / zero load per step serves both (else one per half-step).
// kKS: k-slices per workgroup.  1: four waves, two workgroups per CU.  2 (plan
// cfg 14, 128-row tiles): eight waves in two slices of four, each slice the
// four-wave kernel over half the workgroup's k-steps with its own activation
// buffers and weight stages (144 KiB of LDS, one workgroup per CU, still two
// waves per SIMD); at the end slice 1 hands its accumulators to slice 0
// through LDS.  For shapes with fewer tiles than two per CU this takes the
// place of split-K across workgroups, whose fp32 partials and reduction
// kernel it avoids.  Both slices run the same number of steps (a slice's
// steps past its range load zeros and add exactly 0), so every wave reaches
// every barrier.
//
// Arguments: the first fourteen SGPRs' worth are what the prologue's
// activation, weight and group computations need (X, QW, the tile and split
// geometry, the grid size nb, SZ and the group reciprocal); the library is
// built to have the dispatch preload them into SGPRs (-mllvm
// -amdgpu-kernarg-preload-count), so those loads wait for no kernel-argument
// load, and the rest are loaded meanwhile.  The grid size is an argument
// rather than a read of the dispatch packet.
template <int kMT, bool kSZ1, int kKS = 1, bool AZ = false>
__global__ __launch_bounds__(kNT * kKS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void stream_kernel(const f16* __restrict__ X, const uint32_t* __restrict__ QW, int M, int N,
                   int K, int KTS, int ldx, int nb, const char* __restrict__ SZ, uint32_t gmagic,
                   int gshift, uint32_t sc_off, uint32_t zr_off, uint32_t sz_bytes, int G, int ldy,
                   const f16* __restrict__ bias, f16* __restrict__ Y, float* __restrict__ part) {
  static_assert(kStages == 4, "stage arrays below are written out for four stages");
  static_assert(kMT == 2 || kMT == 4 || kMT == 8, "8-row activation loads per wave");
  static_assert(kKS == 1 || (kKS == 2 && kMT == 8), "two k-slices: 128-row tiles");
  constexpr int kW = kWaves * kKS;       // waves per workgroup
  constexpr int kBM = 16 * kMT;          // rows per workgroup tile
  constexpr int kRPW = kBM / kWaves;     // activation rows each wave streams
  constexpr int kAL = kRPW / 8;          // its 8-row loads per step
  // dequant VALU per MFMA in the interleave: ~64 per half-step over its MFMAs
  constexpr int kVPM = 64 / (kMT * kNTiles);
  // activation buffers: [slice][row][8 octet slots], slot = octet ^ ((row / 2) % 8)
  __shared__ uint4 As0[kKS * kBM * 8], As1[kKS * kBM * 8];
  // weight stages, one array each (the compiler tracks at most 8 LDS-direct
  // targets for its waits; 2 + 4 arrays stay within that):
  //   [wave][half][lane] 16-byte word quads, then
  //   [wave][half][column quad] (scales 0-1, scales 2-3, zeros 0-1, zeros 2-3)
  constexpr int kStageQ = kW * 128;                     // word-quad part (uint4)
  constexpr int kStage = kStageQ + kW * 2 * 16;         // + scale / zero part (uint4)
  __shared__ uint4 St0[kStage], St1[kStage], St2[kStage], St3[kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // 0 .. kW - 1
  const int wv = wave % kWaves;                // position along N
  const int slice = wave / kWaves;             // k-slice (kKS == 2)
  const int l16 = lane & 15;    // column quad (B) / row (A) within a tile
  const int oct = lane >> 4;    // k-octet within a 32-k half-step

  // XCD-aware grouped tile order: the hardware deals workgroups to the 8 XCDs
  // round-robin; each XCD takes a contiguous run of an order that walks kGroupM
  // M-tiles x all N-tiles per group, so concurrent tiles share A rows and B
  // columns in that XCD's L2.  With split-K the grid is tiles x splits and
  // workgroup (tile T, split sp) owns k-steps [sp*KTS, (sp+1)*KTS).
  const int ntn = (N + kBN - 1) / kBN;
  const int ntm = (M + kBM - 1) / kBM;
  const int total = ntn * ntm;
  int B = (int)blockIdx.x;
  if ((nb & 7) == 0) B = (B & 7) * (nb >> 3) + (B >> 3);
  const int sp = B / total;
  const int T = B - sp * total;
  const int group = T / (kGroupM * ntn);
  const int first_m = group * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int rem = T - group * kGroupM * ntn;
  const int m0 = (first_m + rem % gsz) * kBM;
  const int n0 = (rem / gsz) * kBN;
  const int wcol = n0 + wv * (16 * kNTiles);     // first column of this wave
  const int ncol = wcol + 4 * l16;               // this lane's 4 columns
  const bool nv = ncol < N;
  const int KP = K >> 3;
  // this slice's k-steps [KS0, KT) of the workgroup's [sp KTS, sp KTS + KTS);
  // with two slices KTS is a whole number of 8-step blocks and each slice
  // runs KTS / 2 steps (steps at or past KT load zeros)
  const int KSL = KTS / kKS;
  const int KS0 = sp * KTS + slice * KSL;
  const int KT = min(K / kBK, KS0 + KSL);
  const int NG = K / G;

  uint32_t magic_mix;
  asm volatile("v_mov_b32 %0, 0x54006400" : "=v"(magic_mix));
  // rows of X lie ldx elements apart; the range ends after row M - 1's K
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, ((uint32_t)(M - 1) * (uint32_t)ldx + (uint32_t)K) * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(QW, (uint32_t)KP * (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(SZ, sz_bytes);
  (void)NG;

  // Activation stream: wave w fills rows kRPW w .. kRPW (w+1) - 1 with kAL
  // loads of 8 rows; lane L writes row r = kRPW w + 8j + L/8, slot L%8, which
  // holds octet (L%8) ^ ((r/2)%8) = (L%8) ^ (L/16) ^ (4 if kRPW w / 8 + j is
  // odd).  Rows at or past M lie beyond the buffer range (M*K*2 bytes) and
  // read as zero.
  const uint32_t a_voff0 =
      ((uint32_t)(lane >> 3) * (uint32_t)ldx + (uint32_t)((lane & 7) ^ (lane >> 4)) * 8u) * 2u;
  const uint32_t a_voff1 =
      ((uint32_t)(lane >> 3) * (uint32_t)ldx + (uint32_t)((lane & 7) ^ (lane >> 4) ^ 4) * 8u) * 2u;
  const uint32_t a_row0 = (uint32_t)(m0 + kRPW * wv) * (uint32_t)ldx * 2u;
  // A fragment of m-tile i, half-step h: row 16i + l16, octet oct + 4h (in
  // this slice's buffer)
  const int a_frag0 = slice * kBM * 8 + l16 * 8 + ((oct) ^ ((l16 >> 1) & 7));
  const int a_frag1 = slice * kBM * 8 + l16 * 8 + ((oct + 4) ^ ((l16 >> 1) & 7));
  // weight word quad of this lane: packed row 4h + oct of a step, columns ncol..+3
  const uint32_t b_off = nv ? ((uint32_t)oct * (uint32_t)N + (uint32_t)ncol) * 4u : kOobOffset;
  // scale / zero load of this lane: column quad lane / 4, part lane % 4 =
  // scales (0, 1) of columns 0-1 / 2-3, zeros (2, 3) of columns 0-1 / 2-3
  const int qcol = wcol + 4 * (lane >> 2) + 2 * (lane & 1);
  const uint32_t q_off =
      qcol < N ? ((lane & 2) ? zr_off : sc_off) + (uint32_t)qcol * 2u : kOobOffset;

  auto as = [&](auto bc) -> uint4* {
    if constexpr (decltype(bc)::value == 0) return As0;
    else return As1;
  };
  auto stage = [&](auto sc) -> uint4* {
    constexpr int s = decltype(sc)::value;
    if constexpr (s == 0) return St0;
    else if constexpr (s == 1) return St1;
    else if constexpr (s == 2) return St2;
    else return St3;
  };
  auto wq = [&](auto sc) -> uint4* { return stage(sc); };
  auto sz = [&](auto sc) -> uint4* { return stage(sc) + kStageQ; };

  // Past this workgroup's k-range (kt >= KT) the loads below take an offset no
  // buffer range holds and write zeros that are never read.
  auto stream_a = [&](auto bc, int kt) {
    uint4* a = as(bc) + slice * kBM * 8 + kRPW * wv * 8;
    const uint32_t kb = (uint32_t)kt * (uint32_t)(kBK * 2);
#pragma unroll
    for (int j = 0; j < kAL; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (lds_void*)(a + 64 * j), 16, ((kRPW / 8 * wv + j) & 1) ? a_voff1 : a_voff0,
          uniform((kt < KT ? a_row0 + (uint32_t)(8 * j) * (uint32_t)ldx * 2u + kb : kOobOffset)), 0,
          0);
  };
  auto stream_w = [&](auto sc, int kt) {
    uint4* w = wq(sc) + wave * 128;
    uint4* q = sz(sc) + wave * 32;
    const bool in = kt < KT;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (lds_void*)(w + 64 * h), 16, b_off,
          uniform(in ? ((uint32_t)kt * 8u + 4u * (uint32_t)h) * (uint32_t)N * 4u : kOobOffset), 0,
          0);
#pragma unroll
    for (int h = 0; h < (kSZ1 ? 1 : 2); ++h) {
      const uint32_t g = div_group((uint32_t)(kt * kBK + 32 * h), gmagic, gshift);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rq, (lds_void*)(q + 16 * h), 4, q_off, uniform(in ? g * (uint32_t)N * 2u : kOobOffset),
          0, 0);
    }
  };

  // Dequant inputs of one half-step: the lane's word quad and the scales /
  // zeros of its 4 columns (u32 index 2 l16 (+ 32 for h = 1)).
  struct In {
    uint4 w;
    uint2 s, z;
  };
  // The lane indices of these reads are hidden from alias analysis: an
  // LDS-direct load's memory operand covers only its first lane's bytes, and a
  // read the compiler could prove disjoint from the stage's first load would
  // not be matched to that stage and would wait for every load in flight.
  int lane_i = lane;
  asm("" : "+v"(lane_i));
  int q_i[2] = {wave * 32 + l16, wave * 32 + 16 + l16};
  asm("" : "+v"(q_i[0]));
  asm("" : "+v"(q_i[1]));
  auto read_in = [&](auto sc, int h, In& in) {
    in.w = wq(sc)[wave * 128 + 64 * h + lane_i];
    const uint4 c = sz(sc)[q_i[kSZ1 ? 0 : h]];
    in.s = make_uint2(c.x, c.y);
    in.z = make_uint2(c.z, c.w);
  };
  auto dequant = [&](const In& in, f16x8 (&b)[kNTiles]) {
    const f16x2 zm = AZ ? f16x2{} : f16x2{(f16)1024.0f, (f16)64.0f};
    const f16x2 z01 = as_h2(in.z.x), z23 = as_h2(in.z.y);
    const f16x2 s01 = as_h2(in.s.x), s23 = as_h2(in.s.y);
    const f16x2 zz[4] = {f16x2{z01.x, z01.x}, f16x2{z01.y, z01.y}, f16x2{z23.x, z23.x},
                         f16x2{z23.y, z23.y}};
    const ColN cn[4] = {{AZ ? zz[0] : zz[0] + zm, s01.x}, {AZ ? zz[1] : zz[1] + zm, s01.y},
                        {AZ ? zz[2] : zz[2] + zm, s23.x}, {AZ ? zz[3] : zz[3] + zm, s23.y}};
    const uint32_t words[4] = {in.w.x, in.w.y, in.w.z, in.w.w};
#pragma unroll
    for (int c = 0; c < kNTiles; ++c) {
      f16x2 d[4];
      dq_word_nat<AZ>(words[c], cn[c], magic_mix, d);
      b[c] = f16x8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
    }
  };

  // 128 accumulators in VGPRs (the AGPR form of the MFMAs made the compiler
  // shuttle accumulators between the two register files and spill).
  f32x4 acc[kMT][kNTiles];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int c = 0; c < kNTiles; ++c) acc[i][c] = f32x4{};

  // The 32 MFMAs of half-step h: 8 m-tiles x 4 n-tiles; one A fragment per
  // m-tile feeds its four MFMAs.
  auto mfma_half = [&](const uint4* A, const f16x8 (&b)[kNTiles]) {
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
      const f16x8 af = __builtin_bit_cast(f16x8, A[i * 16 * 8]);
#pragma unroll
      for (int c = 0; c < kNTiles; ++c)
        acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, b[c], acc[i][c], 0, 0, 0);
    }
  };
  // Schedule of one half-step region: each MFMA followed by two VALU
  // instructions of the next half-step's dequant (the LDS reads are left to
  // the scheduler: pinning them too lengthened live ranges into spills).
  auto interleave = [&]() {
#pragma unroll
    for (int i = 0; i < kMT * kNTiles; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, kVPM, 0);
    }
  };

  // One k-step (stage s, activation buffer s % 2), software-pipelined: on
  // entry `bf` holds half-step 0's B fragments and `in1` half-step 1's inputs.
  //   start: request step kt+1's activations, then step kt+3's weights;
  //   half 0: MFMAs with bf || dequant in1 -> bn, read step kt+1 half 0 inputs;
  //   half 1: MFMAs with bn || dequant those -> bf, read step kt+1 half 1 inputs;
  //   end: wait for this wave's activation loads, barrier.
  f16x8 bf[kNTiles];
  In in1;
  auto step = [&](auto sc, int kt) {
    constexpr int s = decltype(sc)::value;
    const std::integral_constant<int, s & 1> cur{};
    const std::integral_constant<int, (s & 1) ^ 1> nxt{};
    const std::integral_constant<int, (s + 1) % kStages> s1{};
    const std::integral_constant<int, (s + 3) % kStages> s3{};
    stream_a(nxt, kt + 1);
    // keep the activation loads ahead of the weight loads in issue order (the
    // vmcnt(4) before the closing barrier relies on it)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    stream_w(s3, kt + 3);
    __builtin_amdgcn_sched_barrier(0);
    f16x8 bn[kNTiles];
    In in0n;
    mfma_half(as(cur) + a_frag0, bf);
    dequant(in1, bn);
    read_in(s1, 0, in0n);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(as(cur) + a_frag1, bn);
    dequant(in0n, bf);
    read_in(s1, 1, in1);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    // this wave's part of step kt+1's activations: only the weight and
    // scale / zero loads issued after it (4, or 3 with kSZ1) may still be in
    // flight
    if constexpr (kSZ1)
      asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    tile_barrier();
  };

  // prologue: step KS0's activations and weights of steps KS0 .. KS0+2 in
  // flight, then step KS0's half-step 0 dequantised and half-step 1's inputs
  stream_a(std::integral_constant<int, 0>{}, KS0);
  stream_w(std::integral_constant<int, 0>{}, KS0);
  stream_w(std::integral_constant<int, 1>{}, KS0 + 1);
  stream_w(std::integral_constant<int, 2>{}, KS0 + 2);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  tile_barrier();
  {
    In in0;
    read_in(std::integral_constant<int, 0>{}, 0, in0);
    read_in(std::integral_constant<int, 0>{}, 1, in1);
    dequant(in0, bf);
  }
  // one trip count for the whole workgroup with two slices (each slice's
  // KSL steps from KS0), the slice's own range with one
  const int kend = kKS == 1 ? KT : KS0 + KSL;
  for (int kb = KS0; kb < kend; kb += kStages) {
    step(std::integral_constant<int, 0>{}, kb);
    step(std::integral_constant<int, 1>{}, kb + 1);
    step(std::integral_constant<int, 2>{}, kb + 2);
    step(std::integral_constant<int, 3>{}, kb + 3);
  }

  if constexpr (kKS == 2) {
    // Slice 1's accumulators to slice 0 through the activation buffers, half
    // the m-tiles per round (16 KiB per wave: [register][lane], no bank
    // conflicts).  The last steps' LDS-direct loads (zeros past the range)
    // are drained first so that none lands on the handed-over values; every
    // wave passes every barrier.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    tile_barrier();
    uint4* xb = (wv < 2 ? As0 : As1) + (wv & 1) * (kMT / 2 * kNTiles * 64);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      if (slice == 1) {
#pragma unroll
        for (int i = 0; i < kMT / 2; ++i)
#pragma unroll
          for (int c = 0; c < kNTiles; ++c)
            xb[(i * kNTiles + c) * 64 + lane] =
                __builtin_bit_cast(uint4, acc[r * (kMT / 2) + i][c]);
      }
      tile_barrier();
      if (slice == 0) {
#pragma unroll
        for (int i = 0; i < kMT / 2; ++i)
#pragma unroll
          for (int c = 0; c < kNTiles; ++c)
            acc[r * (kMT / 2) + i][c] += __builtin_bit_cast(f32x4, xb[(i * kNTiles + c) * 64 + lane]);
      }
      if (r == 0) tile_barrier();   // round 1 overwrites what round 0 handed over
    }
    if (slice == 1) return;
  }

  const int rbase = m0 + 4 * oct;
  if (part) {
    if (!nv) return;
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rbase + 16 * i + r;
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
      const int row = rbase + 16 * i + r;
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
        // non-temporal: Y is written once and never read here, so it need not
        // displace the A / B slices in L2 (measured on MI355X: C4 M=4096 397.9
        // -> 396.5 us, M=2048 215.6 -> 214.9 us, medians of 5)
        __builtin_nontemporal_store(o, reinterpret_cast<f16x4*>(Y + (size_t)row * ldy + ncol));
      }
    }
  }
}

// k-steps per split: whole 4-step blocks per k-slice
int split_steps(int K, int split, int slices) {
  const int KT = K / kBK;
  const int unit = kStages * slices;
  return ((KT + split - 1) / split + unit - 1) / unit * unit;
}

template <int kMT, bool kSZ1, int kKS, bool AZ>
hipError_t launch_kernel(const GemmArgs& a, int split, float* part, hipStream_t st) {
  constexpr int kBM = 16 * kMT;
  const int tiles = ((a.N + kBN - 1) / kBN) * ((a.M + kBM - 1) / kBM);
  const int KT = a.K / kBK;
  // never more splits than occ2_splits() gives for the same request, so
  // occ2_workspace_bytes() covers the partials
  const int kts = split_steps(a.K, split, kKS);
  const int nsplit = split > 1 ? (KT + kts - 1) / kts : 1;   // every split non-empty
  // unsplit with two slices: whole 8-step blocks (steps past KT load zeros)
  const int kts1 = (KT + kStages * kKS - 1) / (kStages * kKS) * (kStages * kKS);
  // scales and zeros through one buffer resource based at the lower address
  const char* sc = static_cast<const char*>(a.sc);
  const char* zr = static_cast<const char*>(a.zr);
  const char* base = sc < zr ? sc : zr;
  const uint32_t sz_bytes = (uint32_t)((sc < zr ? zr : sc) - base) +
                            (uint32_t)(a.K / a.G) * (uint32_t)a.N * 2u;
  const GroupDiv gd = group_div(a.G);
  hipLaunchKernelGGL((stream_kernel<kMT, kSZ1, kKS, AZ>), dim3(tiles * nsplit), dim3(kNT * kKS), 0, st,
                     static_cast<const f16*>(a.x), reinterpret_cast<const uint32_t*>(a.qw), a.M, a.N,
                     a.K, nsplit > 1 ? kts : kts1, a.ldx, tiles * nsplit, base, gd.magic, gd.shift,
                     (uint32_t)(sc - base), (uint32_t)(zr - base), sz_bytes, a.G, a.ldy,
                     static_cast<const f16*>(a.bias), static_cast<f16*>(a.y),
                     nsplit > 1 ? part : nullptr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  return launch_splitk_reduce(part, a.bias, a.y, a.M, a.N, a.ldy, nsplit, st);
}

template <int kMT, int kKS, bool AZ>
hipError_t launch_wz(const GemmArgs& a, int split, float* part, hipStream_t st) {
  return a.G % (2 * 32) == 0 ? launch_kernel<kMT, true, kKS, AZ>(a, split, part, st)
                             : launch_kernel<kMT, false, kKS, AZ>(a, split, part, st);
}

template <int kMT, int kKS = 1>
hipError_t launch_wg(const GemmArgs& a, int split, float* part, hipStream_t st) {
  return a.any_zeros ? launch_wz<kMT, kKS, true>(a, split, part, st)
                     : launch_wz<kMT, kKS, false>(a, split, part, st);
}

}  // namespace

int stream_splits(int K, int split, int slices) {
  if (split <= 1 || K / kBK <= 1) return 1;
  const int kts = split_steps(K, split, slices);
  return (K / kBK + kts - 1) / kts;
}

bool stream_gemm_applicable(int M, int N, int K, int G) {
  return occ2_gemm_applicable(M, N, K, G) && K % (kBK * kStages) == 0;
}

// rows x 256 tiles, rows = 128, 64 or 32; two k-slices per workgroup only
// with 128 rows.  Same applicability and split rule as the two-waves-per-SIMD
// register kernel, plus K % 256 == 0.  Scales and zeros further than 2 GiB
// apart (one buffer resource cannot span them) take that register kernel
// (128 x 256 tiles, same results up to fp32 summation order inside an MFMA).
hipError_t launch_stream_gemm(const GemmArgs& a, int rows, int split, float* part,
                              hipStream_t st, int slices) {
  if (!stream_gemm_applicable(a.M, a.N, a.K, a.G)) return hipErrorInvalidValue;
  if (occ2_splits(a.K, split) > 1 && !part) return hipErrorInvalidValue;
  const uintptr_t sc = reinterpret_cast<uintptr_t>(a.sc), zr = reinterpret_cast<uintptr_t>(a.zr);
  const uint64_t dist = sc < zr ? zr - sc : sc - zr;
  const uint64_t bytes = (uint64_t)(a.K / a.G) * (uint64_t)a.N * 2u;
  if (dist + bytes >= (1ull << 31)) return launch_occ2_gemm(a, split, part, st);
  if (slices == 2) return rows == 128 ? launch_wg<8, 2>(a, split, part, st) : hipErrorInvalidValue;
  switch (rows) {
    case 128: return launch_wg<8>(a, split, part, st);
    case 64: return launch_wg<4>(a, split, part, st);
    case 32: return launch_wg<2>(a, split, part, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace w4a16
