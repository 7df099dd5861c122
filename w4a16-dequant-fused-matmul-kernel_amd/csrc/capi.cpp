// extern "C" entry points of libw4a16.so (declared in include/w4a16.h).
//
// Host-side argument checks mirror the reference's preconditions
// (w4a16-kernel/src/w4a16/triton_kernel.py:153-182, cuda/w4a16_gemm.cu:80-96,
// quant.py:114-119) but report status codes instead of raising; the Python
// package maps them to the reference's exception types.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <mutex>
#include <vector>

#include "../../include/w4a16.h"
#include "w4a16_launch.h"

using namespace w4a16;

namespace {

constexpr int kMaxDevices = 64;
constexpr int kDefaultCUs = 256;  // MI355X; used only if the device cannot be queried
std::atomic<int> g_cu_count[kMaxDevices];

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return kDefaultCUs;
  }
  int c = g_cu_count[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = kDefaultCUs;
  }
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

bool fits_i32(int64_t v) { return v >= 0 && v <= INT32_MAX; }

int check_gemm_shape(int64_t M, int64_t N, int64_t K, int64_t G) {
  if (!fits_i32(M) || !fits_i32(N) || !fits_i32(K)) return W4A16_ERR_BAD_SHAPE;
  if (K % 8 != 0) return W4A16_ERR_BAD_SHAPE;
  if (G <= 0 || G > INT32_MAX || K % G != 0) return W4A16_ERR_BAD_GROUP;
  // element counts must stay addressable with size_t and kernel int math on rows
  if ((uint64_t)M * (uint64_t)K > (1ull << 46) || (uint64_t)M * (uint64_t)N > (1ull << 46) ||
      (uint64_t)K * (uint64_t)N > (1ull << 48))
    return W4A16_ERR_BAD_SHAPE;
  return W4A16_OK;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool gemv_applicable(int64_t M, int64_t N, int64_t G) {
  return M >= 1 && M <= kGemvMaxM && N % 4 == 0 && G % 32 == 0;
}
bool mfma_applicable(int64_t N, int64_t G) { return N % 4 == 0 && G % 32 == 0; }
bool skinny_applicable(int64_t M, int64_t G) { return M >= 1 && M <= kSkinnyMaxM && G % 32 == 0; }
bool fits(int64_t M, int64_t N, int64_t K, int64_t G) {
  return operands_fit((int)M, (int)N, (int)K, (int)G);
}

// Widest column block that still gives every CU a workgroup; split K across
// workgroups only when even 16-column blocks cannot fill the device.
// GEMV column block (measured on MI355X, M = 1 and 2): the widest block that
// still gives every CU a workgroup; for K < 8192 (no split), where 16-column
// blocks would leave the CUs between one and two blocks each, 32-column blocks
// (at most one per CU) win (K = 4096, N = 6144: 7.3 -> 6.5 us at M = 1, 9.0 ->
// 7.5 us at M = 2).
// Where 16-column blocks would leave the CUs between one and two blocks each
// (4096 < N <= 8192 on MI355X): 32-column blocks (at most one per CU), at any K
// and unsplit.  Measured on MI355X, M = 1, µs, against 16-column blocks:
// K = 4096, N = 6144 7.3 -> 6.5; K = 8192, N = 5120 / 6144 12.66 / 12.78 ->
// 9.64 / 9.70; K = 13824 19.86 / 20.22 -> 14.72 / 14.73 (split 4 ways: 18.9,
// 8 waves: 15.8); M = 2, K = 8192, N = 6144 15.38 -> 11.29.
bool gemv_band32(int64_t N, int cus) {
  const int64_t b16 = (N + 15) / 16;
  return b16 > cus && b16 <= 2 * (int64_t)cus;
}

// M <= 2, K > 2048, where 32-column blocks would outnumber the CUs but
// 64-column ones would not (8192 < N < 16384 on MI355X): 64-column blocks
// with staged activations and the dot products on the matrix cores (cfg 7),
// unsplit (the skinny kernel's 64-column blocks instead for K <= 4096 where
// they apply: decode_takes_skinny).  The 32-column blocks take more than one
// round there.  Measured on MI355X, µs, against 32-column blocks: M = 1,
// K = 8192, N = 10240 17.39 -> 12.76; N = 14336 18.21 -> 13.84; M = 2,
// K = 8192, N = 11008 20.78 -> 12.85; K = 14336, N = 12288 27.29 -> 19.81;
// M = 1, K = 4096, N = 11008 11.03 -> 8.37 (skinny 7.82); K = 2048 slower
// (5.57 -> 6.14).
bool gemv_band64(int64_t M, int64_t N, int64_t K, int cus) {
  return M <= 2 && K > 2048 && (N + 31) / 32 > cus && (N + 63) / 64 < cus;
}

int gemv_cols_auto(int64_t M, int64_t N, int64_t K, int cus) {
  // M <= 2: 128-column blocks where they give at least 7/8 of the CUs one
  // each (N = 28672 on MI355X: 224), a workgroup per CU reading two 256-byte
  // segments of each packed row (measured on MI355X with the dot products on
  // the matrix cores, cfg 7, against 64-column blocks: M = 1, K = 8192,
  // N = 28672 25.0 vs 25.9 us; K = 4096 15.0 vs 15.9; M = 2, K = 8192 25.0 vs
  // 26.1)
  // (and at most one each: N = 37888, 296 blocks, took 25.9 us at K = 3584
  // against 21.7 on 64-column blocks, 45.1 against 37.9 at K = 8192), and
  // down to where 64-column blocks would take more than one round (N > 16384
  // on MI355X: M = 1, K = 4096, N = 18432 / 20480 / 24576 14.84 / 14.80 /
  // 15.46 -> 13.69 / 13.68 / 14.47 us; K = 8192 24.22 / 24.38 / 25.06 ->
  // 22.16 / 22.93 / 23.91; M = 2, K = 8192, N = 20480 24.60 -> 23.02), unsplit
  if (M <= 2 && (N + 127) / 128 <= cus && (N + 63) / 64 > cus) return 128;
  if (gemv_band64(M, N, K, cus)) return 64;
  static const int kCols[] = {256, 64, 32, 16};
  for (int c : kCols)
    if ((N + c - 1) / c >= cus) return c == 16 && gemv_band32(N, cus) ? 32 : c;
  return 16;
}

// GEMV waves per workgroup and activation staging (measured on MI355X with
// the sweep-ordered direct kernel for M <= 2, medians of 3 runs of 60 calls):
//   * 64-column blocks stage the activations in LDS: 16 lanes share a row,
//     and one load and one permute per element beat one per lane (M = 1, K =
//     4096, N = 28672: 16.2 us against 18.6 direct; M = 1, K = 8192, N = 28672:
//     27.9 against 32.3; M = 2 likewise), with the dot products on the matrix
//     cores (cfg 7, 8 waves; gemv.hip); 256-column blocks the same with dot2
//     (cfg 4), 128-column blocks with 16 waves (cfg 5);
//   * 16- and 32-column blocks read them directly with 16 waves (cfg 2) at
//     M = 1 for any K (K = 28672, N = 8192: 27.2 us against 30.8 with 8 waves
//     and 28.7 staged; K = 14336, N = 4096: 11.9 against 13.9 with 8 waves;
//     32-column blocks, K = 4096, N = 6144: 6.43 against 7.19), except
//     16-column blocks with 2048 < K <= 4096 at M = 1, where 8 waves with four
//     rows per lane do better (C2: 4.66 against 4.75 us, G = 64 4.81 against
//     4.92; N = 2048 and K = 2048 a tie), and at M = 2 up to K / split =
//     8192, with 8 waves (cfg 1) beyond;
//   * M > 2 always stages them (gemv_kernel, cfg 1).
int gemv_waves_cfg(int64_t M, int64_t K, int split, int cols) {
  const int64_t ks = K / (split > 0 ? split : 1);
  if (M > 2) return kGemvDefaultConfig;
  const bool stage = split <= 1 && ks <= 16384 && cols >= 64;
  // 64- and 128-column blocks: the dot products on the matrix cores (cfg 7,
  // 8 waves; measured on MI355X against the dot2 kernel's best, 16 waves on
  // 128-column blocks: M = 1, K = 8192, N = 28672 25.0 vs 26.3 us, G = 32 25.8
  // vs 26.3, K = 4096 15.0 vs 15.1; M = 2, K = 8192 25.0 vs 30.6, K = 4096
  // 15.2 vs 17.2)
  if (cols == 128 || (stage && cols == 64)) return kGemvDefaultConfig + 6;
  if (stage) return kGemvDefaultConfig + 3;
  if (M == 1 && cols == 16 && ks > 2048 && ks <= 4096) return kGemvDefaultConfig;
  return (M == 1 || ks <= 8192) ? 2 : kGemvDefaultConfig;
}

// GEMV k-split by shape (measured on MI355X, M = 1..8, fp32 partials plus the
// split-order reduction kernel): with K >= 8192 and fewer column blocks than
// CUs, four splits win 12-50 % (K = 14336, N = 1024: 11.7 -> 7.3 us;
// K = 28672, N = 1024: 20.5 -> 10.0 us); at K = 4096 the extra pass costs more
// than the extra workgroups recover (4.6 -> 5.4 us); at (nearly) one block per
// CU it is neutral to 3 % slower; 3 or 6 splits, whose row ranges cut
// quantisation groups, lose to 4.
int gemv_split_auto(int64_t N, int64_t K, int cols, int cus) {
  const int64_t nblk = (N + cols - 1) / cols;
  return (K / 8 >= 1024 && nblk < cus * 7 / 8) ? 4 : 1;
}

// Long rows at M <= 2 (K >= 16384 for M = 1, K >= 12288 for M = 2) on
// 32 .. 7/8-of-the-CUs 64-column blocks: the dot products on the matrix cores
// (cfg 7), K split into the fewest powers of two (at most 8) that give 7/8 of
// the CUs a workgroup, one reduction pass.  Measured on MI355X against the
// plans these shapes had (16/32-column dot2 blocks): M = 1, K = 28672,
// N = 8192 27.4 -> 24.6 us (split 2); N = 4096 19.9 -> 16.4 (4); N = 2048 15.8
// -> 12.2 (8); M = 2, K = 28672, N = 8192 39.3 -> 26.9; K = 14336, N = 4096
// 16.0 -> 11.6.  Shorter rows lose the reduction pass's cost (M = 1, K = 8192,
// N = 8192 10.6 -> 11.3 us; K = 14336, N = 8192 15.8 -> 16.3).  Returns the
// split, or 0 where the rule does not apply.
int gemv_mfma_split(int64_t M, int64_t N, int64_t K, int cus) {
  if (M > 2 || K < (M == 2 ? 12288 : 16384)) return 0;
  // M = 1 where 32-column blocks are fewer than the CUs (4096 < N < 8192):
  // those, unsplit (K = 16384, N = 6144: 16.4 against 18.0 us; K = 28672
  // 25.4 against 27.1; K = 20480, N = 5120 19.2 against 22.0; not at N = 8192,
  // one full round: 27.0 against 24.8, nor at M = 2: 19.4 against 18.2)
  if (M == 1 && gemv_band32(N, cus) && (N + 31) / 32 < cus) return 0;
  const int64_t nblk = (N + 63) / 64;
  const int64_t want = (int64_t)cus * 7 / 8;
  if (nblk < 32 || nblk >= want) return 0;
  int s = 2;
  while (nblk * s < want && s < 8) s *= 2;
  return s;
}

// Prefill tile configuration by shape (measured on MI355X, C4/C5 shapes):
//   * the 128 x 256 two-waves-per-SIMD 16x16x32 kernel with activations and
//     weights streamed into LDS (cfg 11, K % 256 == 0) wherever the tiles fill
//     half the CUs or M >= 1024: 5-8 % faster than cfg 7 at C4 M = 4096,
//     15-20 % at M = 512 and at C5 M = 256; without K % 256 == 0, cfg 7 for
//     M >= 1024 and the 32x32x16 two-waves kernel (cfg 6) for the rest;
//   * fewer tiles (short M, narrow N): cfg 11 split along K for about two
//     workgroups per CU (cfg 7 for one per CU where K % 256 != 0; fp32
//     partials + one reduction kernel), when K allows at least 8 k-steps per
//     split; else narrow 32 x 512 tiles (cfg 2) or the one-wave 128 x 256
//     (cfg 1);
//   * M <= 64: the same streamed kernel with 32-row (M <= 32, cfg 12) or
//     64-row tiles (cfg 13), split likewise (small_m_takes_stream below says
//     when it beats the skinny and decode kernels).
struct MfmaChoice {
  int cfg, split;
};

bool skinny_quad(int64_t M, int64_t N, int64_t K, int64_t G, int cus);

// Decode batches 3 <= M <= 8: the MFMA skinny kernel does the M dot products
// per dequantised pair on the matrix cores where the GEMV spends M v_dot2 on
// each; measured on MI355X it wins from M = 3 up to N = 16384 (M = 8,
// K = N = 4096: 7.7 vs 12.1 us; M = 3, K = 14336, N = 4096: 17.2 vs 20.8 us;
// M = 4, K = 4096, N = 6144: 9.7 vs 11.5 us) and from M = 5 on wider weights
// (M = 5, K = 4096, N = 28672: 29.7 vs 32.6 us).  At M <= 4 on wider weights
// the skinny kernel's 64-column blocks win at any K where they apply
// (skinny_quad; M = 3, K = 4096, N = 28672: 18.3 vs 22.0 us; G = 64 / 32:
// 17.8 / 20.2 vs 21.9 / 22.3; N = 37888, G = 64 / 32: 23.5 / 27.3 vs 30.1 /
// 30.7; K = 5120 / 6144 / 8192, N = 27648 / 28672 / 28672: 21.1 / 24.8 /
// 30.8 vs 26.0 / 33.8 / 43.4; K = 8192, N = 16896 26.1 vs 40.0; G = 64,
// K = 8192, N = 28672 33.7 vs 44.6), else the GEMV (its 32-column blocks:
// G = 32, K = 5120, N = 27648: 30.7 vs 25.9).  Few column blocks with long K
// take the GEMV split along K: where 16-column blocks would give at most a
// quarter of the CUs one (N <= 1024 on MI355X) from K = 8192, at most half
// (N <= 2048) from K = 16384 at M <= 4 (M = 3 / 4 / 5 / 6 / 8, K = 16384,
// N = 1024: 8.9 / 9.4 / 11.9 / 12.7 / 14.0 vs 14.7 / 14.7 / 14.7 / 15.0 /
// 16.1 us; K = 8192, M = 3 / 6: 7.8 / 8.6 vs 8.8 / 9.2, M = 8 9.5 vs 10.0 the
// other way; N = 2048, K = 16384, M = 3 / 4: 11.4 / 12.4 vs 14.9 / 15.0, M = 5
// 15.0 vs 16.1 the other way; G = 32 / 64, M = 4, N = 2048: 12.6 / 12.4 vs
// 21.9 / 17.9).
// M <= 2, K > 2048: the skinny kernel (MFMA dots, one batch per wave up to
// K = 4096) where the GEMV's blocks fit the CUs badly (measured on MI355X, µs,
// against the GEMV's plan):
//   * 32-column blocks where 16-column ones outnumber the CUs but 32-column
//     ones do not (4096 < N <= 8192), up to K = 4096 (one batch per wave; any
//     G), and at M = 2 with G % 128 == 0 up to K = 8192, against the GEMV's
//     32-column blocks: M = 1, K = 4096, N = 4608 / 6144 / 8192: 6.25 / 6.45 /
//     6.61 -> 6.02 / 6.17 / 6.29; K = 3584, N = 6144 6.35 -> 6.05; M = 2,
//     K = 4096, N = 6144 / 8192 7.52 / 7.79 -> 6.33 / 6.50, K = 5120 9.51 ->
//     8.56, K = 8192 a tie (M = 1, K = 5120 .. 13824: the GEMV's blocks 5-15 %
//     faster; 1024 < K <= 2048 slower: 4.06 -> 4.41; K <= 1024 faster:
//     K = 1024, N = 5120 / 8192 3.97 / 3.94 -> 3.51 / 3.51, M = 2 4.60 /
//     4.66 -> 3.61 / 3.68).  Smaller groups, N = 6144:
//     M = 2, K = 3584 / 4096, G = 64: 7.57 / 7.57 -> 6.43 / 6.50, G = 32:
//     7.66 / 7.68 -> 6.78 / 6.81; M = 1 G = 64 6.43 / 6.50 -> 6.22 / 6.37,
//     G = 32 a tie; K = 5120 the GEMV's (M = 2, G = 64: 9.63 vs 10.17);
//   * G % 128 == 0: 64-column blocks with K <= 4096 in the 64-column band of
//     gemv_band64
//     (M = 1, K = 4096, N = 9216 / 11008 / 14336: 8.30 / 8.37 / 8.69 ->
//     7.71 / 7.77 / 8.42; M = 2, N = 14336 8.85 -> 8.59) and where 128-column
//     blocks would outnumber the CUs but 256-column ones would not fill them
//     (M = 1, K = 3584 / 4096, N = 37888: 21.7 / 22.5 -> 20.9 / 21.3; M = 2,
//     K = 4096 22.7 -> 21.8; from N = 65536 the GEMV's 256-column blocks fill
//     the CUs; G = 64 a tie, G = 32 the GEMV's: K = 4096, N = 11008 8.54
//     vs 9.67);
//   * K <= 2048 outside the 32-column band: every workgroup's single batch
//     is short, and the skinny kernel's 16- / 64-column blocks beat the
//     GEMV's (M = 1, K = 2048, N = 2048 / 4096 / 16384 / 28672: 3.92 / 4.00 /
//     6.61 / 10.28 -> 3.60 / 3.70 / 5.75 / 8.70; M = 2 4.50 / 4.63 / 6.70 /
//     10.34 -> 3.78 / 3.94 / 5.85 / 8.87; K = 1024 20-35 % faster; G = 64
//     alike; G = 32 only on 16-column blocks: M = 2, N = 4096 4.66 -> 4.17,
//     64-column blocks a tie).
bool decode_takes_skinny(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  if (!skinny_applicable(M, G)) return false;
  const int64_t b16 = (N + 15) / 16;
  if (M <= 2) {
    const bool wide32 = N % 2 == 0 && b16 > cus && (N + 31) / 32 <= cus;
    if (wide32) return K <= 1024 || (K > 2048 && K <= (M == 2 && G % 128 == 0 ? 8192 : 4096));
    if (K <= 2048) return b16 <= cus || G % 64 == 0;
    return K <= 4096 && G % 128 == 0 && skinny_quad(M, N, K, G, cus) &&
           (gemv_band64(M, N, K, cus) || ((N + 127) / 128 > cus && (N + 255) / 256 < cus));
  }
  if (M > kGemvMaxM) return false;
  if ((K >= 8192 && b16 * 4 <= cus) || (K >= 16384 && M <= 4 && b16 * 2 <= cus)) return false;
  return N <= 16384 || M >= 5 || skinny_quad(M, N, K, G, cus);
}

// Small batches (4 <= M <= 64) on large enough weights: the streamed prefill
// kernel with 32-row (M <= 32) or 64-row tiles (cfg 12 / 13), split along K
// for about 448 workgroups, beats the skinny kernel and the decode GEMV
// (measured on MI355X against each one's best plan): M = 8, K = 8192, N =
// 28672: 37.2 vs 57.6 us; M = 16, K = 4096, N = 28672: 23.5 vs 38.9 (and vs
// 67 for the skinny kernel); M = 32, K = 14336, N = 4096: 23.5 vs 31.9; M = 64,
// K = 4096, N = 14336: 24.6 vs 70.5; M = 4, K = 28672, N = 8192: 40.0 vs 47.2.
// Its fixed cost (a split-K pass, K-steps of 64) loses on small weights, and
// the skinny kernel's cost grows with M, so the size threshold falls with M:
// M = 16 keeps the skinny kernel at K = 14336, N = 4096 (20.3 vs 22.4) and
// below 20 MB; M = 9 wins only from N = 14336 (16.9 vs 18.1); M <= 3 keeps the
// GEMV (M = 3, K = 4096, N = 28672: 21.9 vs 22.7).
// Long rows on 16-column skinny blocks (N <= 4096 here; wider weights take the
// skinny kernel's 32- / 64-column blocks, which pass X once per 32 / 64
// columns, through the size rules and the skinny branch of make_plan): a
// workgroup's time grows with K x M (every block streams all of X), the split
// streamed tiles' with the weight bytes, so from M = 9 at K >= 24576, from
// M = 16 beyond K = 16384, and beyond K = 8192 with smaller groups (G = 32
// from M = 16, G = 64 from M = 17) the streamed tiles win (measured on MI355X,
// µs, N = 4096, skinny vs streamed): K = 28672, G = 128, M = 12 / 16 / 17 / 20:
// 31.0 / 33.2 / 37.6 / 37.6 vs 28.1 / 28.6 / 28.9 / 29.3 (G = 64: 32.2 / 36.4
// / 40.5 / 44.7 vs 28.3 / 28.2 / 28.6 / 29.2); K = 20480, M = 16: G = 128 a
// tie, G = 64 27.1 vs 24.9; G = 32, M = 16, K = 11008 / 14336: 19.8 / 23.5 vs
// 18.3 / 22.3, M = 17 / 20, K = 14336 / 11008: 25.1 / 23.0 vs 22.3 / 19.2;
// G = 64, M = 17, K = 14336: 22.7 vs 22.1.  Kept on the skinny kernel: M <= 8
// (K = 28672, M = 4 / 8, G = 128: 24.4 / 27.0 vs 28.6 / 27.7; K = 20480,
// M = 8: 20.7 vs 24.2), M = 16 at K = 14336 (G = 64: 20.2 vs 22.0), K = 8192
// (G = 32, M = 16: 15.3 vs 16.8).
bool small_m_takes_stream(int64_t M, int64_t N, int64_t K, int64_t G) {
  if (M < 4 || M > kSkinnyMaxM) return false;
  if (!mfma_cfg_applicable(12, (int)M, (int)N, (int)K, (int)G)) return false;
  const int64_t mb = K / 2 * N >> 20;   // packed weight MiB
  if (M >= 48) return true;
  if (M >= 9 && K >= 24576) return true;
  if (M >= 16 && K > (G % 128 == 0 || (G % 64 == 0 && M == 16) ? 16384 : 8192)) return true;
  if (M >= 24) return mb > 8;
  if (M >= 16) return N >= 8192 && mb >= 20;
  return (N >= 14336 && mb >= 24) || mb >= 64;
}

// The skinny kernel's 32-column blocks (two columns per lane, N even, M <= 32)
// where 16-column blocks would put two on some CUs: one activation stream and
// 8-byte weight loads per 32 columns (measured on MI355X against 16-column
// blocks, K = 4096, N = 6144: M = 4 / 8 / 16 / 32 8.3 / 8.5 / 9.4 / 13.0 vs
// 9.2 / 10.1 / 12.4 / 19.1 us; at N = 4096, 128 blocks for 256 CUs, slower:
// M = 4 8.2 vs 6.4).
bool skinny_wide(int64_t M, int64_t N, int cus) {
  return M <= 32 && N % 2 == 0 && (N + 15) / 16 > cus;
}

// ... and it beats the streamed small-M tiles up to N = 8192, and to N = 16384
// for M <= 16 (measured on MI355X: M = 24, K = 4096, N = 6144: 11.9 vs 14.6
// us; M = 4, K = 28672, N = 8192: 34.1 vs 38.9; M = 12, K = 4096, N = 14336:
// 15.3 vs 17.2), not on wider weights, whose 256-column streamed tiles share
// the activations (M = 16, K = 4096, N = 28672: 27.8 vs 23.8; M = 32,
// N = 14336: 22.6 vs 19.6).  Measured with G = 128; smaller groups add
// scale / zero loads to every skinny k-step and lose (M = 16, K = 28672,
// N = 8192: G = 32 55.1 vs 48.6 us, G = 64 48.1 vs 46.1; G = 128 a tie).
// Beyond M = 16 up to K = 8192 (M = 17 / 20, K = 8192, N = 8192: 17.1 / 18.2
// vs 20.7 / 20.9; M = 20, K = 6144, N = 8192: 17.8 vs 20.4; K = 8192,
// N = 6144: 15.2 vs 19.6); longer rows with all M rows in each workgroup
// gain nothing (M = 17, K = 14336, N = 8192: 26.1 vs 25.7) or lose (16-row
// groups on the same blocks already do: M = 32, N = 6144, K = 14336: 39.0 vs
// 25.6; N = 8192, K = 28672: 75.4 vs 44.0).
// Smaller groups at M <= 16 up to K = 8192 and N = 8192 as well (planner
// audit, µs: M = 16, K = N = 8192: G = 64 19.2 -> 16.6, G = 32 19.9 ->
// 18.5; not N = 10240, where the whole-row 32-column blocks lose to 16-row
// groups on 64-column blocks and to the streamed tiles: G = 32, M = 16
// 31.0 against 23.5).
bool skinny_wide_beats_stream(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  return skinny_wide(M, N, cus) && (G % 128 == 0 || (K <= 8192 && M <= 16 && N <= 8192)) &&
         (M <= 16 || K <= 8192) &&
         (N <= 8192 || (N <= 16384 && M <= 16));
}

// 64-column blocks (four columns per lane: 16-B weight loads, one activation
// stream per 64 columns) for M <= 16 where they still give more than half the
// CUs a block (N > 8192 on MI355X), with G % 64 == 0, or any G with K <= 4096
// (one batch per wave, whose scale / zero loads are few).  Measured there
// against the best other plan (µs): M = 4 / 8, K = 4096, N = 28672: 20.9 /
// 22.4 vs 22.3 / 23.6 (streamed tiles; G = 64: 18.3 / 19.5 vs 22.4 / 22.8;
// G = 32: 20.7 / 22.1 vs 23.2 / 23.6); M = 8, K = 8192, N = 28672: 35.6 vs
// 40.1 (G = 64: 35.9 vs 38.4); M = 4: G = 64 34.1 vs 42.7; M = 16, K = 4096,
// N = 14336: 14.7 vs 16.4 (32-column blocks; G = 64 / 32: 11.1 / 12.9 vs
// 17.1 / 17.6 streamed); M = 16, K = 4096, N = 28672: 23.7 vs 23.3 (G = 64:
// 21.8 vs 23.9); long rows: M = 8, K = 28672, N = 16384: 57.2 vs 67.9;
// M = 12 / 16, K = 14336, N = 14336: 29.6 / 31.0 vs 38.8 / 34.6; M = 12,
// K = 8192, N = 16384, G = 64: 22.8 vs 27.1.  Fewer blocks lose (K = 28672,
// N = 8192: 52.5 vs 43.4), and so does G = 32 with K > 4096 (K = 8192,
// N = 28672, M = 4 / 8: 39.9 / 41.3 vs 38.9 / 39.2; M = 8, K = N = 14336:
// 38.4 vs 34.3).
// Beyond two blocks per CU at M > 8 the streamed 32-row tiles win (M = 16,
// K = 8192, N = 57344, 896 blocks: 69.6 vs 65.7 split 2; 448 blocks,
// N = 28672, K = 4096 / 5120: 20.1 / 25.2, the best plan).
// Smaller groups also up to K = 6144 where the blocks take one round
// (planner audit, G = 32, µs: M = 4 / 8 / 16, K = 5120, N = 15360: 20.6 /
// 21.2 / 23.3 on the streamed tiles -> 17.8 / 18.1 / 18.3; not N = 27648:
// 28.1 / 29.1 / 32.3 against 26.1 / 26.4 / 27.3 streamed).
bool skinny_quad(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  const int64_t b64 = (N + 63) / 64;
  return M <= 16 && N % 4 == 0 && (G % 64 == 0 || K <= 4096 || (K <= 6144 && b64 <= cus)) &&
         b64 > cus / 2 && (M <= 8 || b64 <= 2 * (int64_t)cus);
}

// Skinny blocks with one 16-row group per workgroup (plan tile_m = 16) for
// 17 <= M <= 64: each workgroup streams 16 rows of X instead of all M, which
// is what bounds the kernel from M = 16 (X's bytes per CU, not the weights'),
// and no cross-workgroup reduction is needed.  The block width keeps the
// workgroups near the CU count: 32 columns while 2 x N / 32 groups fit the
// CUs, else 64 columns up to two rounds (K <= 4096, one batch per wave); with
// longer K (the 4-wave loop) only two row groups on one round, 64-column
// blocks from M = 24 (a 17th row alone costs a second weight pass there).
// Three or four row groups with K > 4096 (G = 128) where their blocks fit one
// round: K = 5120 / 8192 / 16384, N = 2048, M = 48 / 64 on 32-column blocks:
// 10.5 / 13.7 / 23.1 and 9.8 / 13.1 / 23.0 vs 15.1 / 18.3 / 25.5 and 15.3 /
// 18.4 / 25.9 on the streamed tiles (M = 33: 13.3 vs 16.8 at K = 8192);
// N = 4096 / 5120, K = 5120 / 8192 on 64-column blocks: M = 48 14.3 / 14.7 /
// 18.5 / 18.7 vs 17.6 / 19.0 / 21.8 / 24.6 (64-column blocks at K = 16384 and
// two rounds slower, as with two groups).  With K <= 4096 the 64-column
// blocks may take more rounds the shorter K is: K = 2048, M = 40 / 48 / 64,
// N = 11008 / 16384 (516-1024 workgroups): 12.1 / 15.4, 12.8 / 15.8, 12.3 /
// 15.4 vs 16.0 / 18.7, 16.7 / 19.8, 17.8 / 21.3; not N = 28672 (1344-1792:
// 22.3-24.9 vs 21.7-23.7), nor K = 4096 beyond two rounds (M = 48 / 64,
// N = 11008: 24.3 / 23.9 vs 22.5 / 22.5).
// Returns the skinny cfg (2 or 3) and rows per workgroup, or cfg -1 for the
// whole-rows plans.  Measured on MI355X against the
// automatic plan before it (µs, G = 128): K = 4096, N = 4096, M = 24 / 32 /
// 48 / 64: 9.60 / 10.91 / 16.17 / 16.57 -> 8.14 / 8.12 / 9.28 / 8.56; N = 6144
// M = 32 / 48: 11.88 / 19.00 -> 9.80 / 15.96; N = 8192 M = 64: 21.16 ->
// 15.84; N = 14336 M = 32: 19.19 -> 17.72; K = 14336, N = 4096, M = 17 / 32:
// 22.10 / 23.49 -> 20.72 / 20.94; N = 6144 / 8192, K = 8192, M = 32: 20.64 /
// 21.49 -> 19.10 / 19.11.  Slower (kept on the streamed tiles): N = 28672 at
// every M (M = 32: 26.4 vs 34.2), three or four row groups with K > 4096
// (M = 48, K = 8192, N = 8192: 25.6 vs 29.4), M = 17 on 64-column blocks with
// K > 4096, and long rows, whose time on a workgroup grows with K while the
// split streamed tiles' grows with the weight bytes: 32-column blocks beyond
// K = 16384 (K = 28672, N = 4096, M = 24 / 32: 38.3 / 39.5 vs 29.6 / 30.4),
// 64-column ones beyond K = 8192 (N = 6144, M = 32, K = 14336 / 28672: 28.3 /
// 49.7 vs 25.6 / 35.3; N = 8192, M = 24, K = 14336 28.6 vs 26.5; M = 32,
// K = 28672: 54.5 vs 44.0; K = 11008 a tie).
// Smaller groups (µs, G = 64 / 32, against the automatic plan before): with
// K <= 4096 the same rules win, except 64-column blocks beyond one round at
// G = 32 (K = 4096, N = 4096, M = 24 / 32 / 48 / 64: 9.71 / 11.01 / 16.36 /
// 16.80 -> 8.34 / 8.40 / 9.85 / 9.31, G = 32 11.01 / 12.63 / 16.74 / 17.24
// -> 8.67 / 9.27 / 11.29 / 10.36; N = 6144, M = 32: 15.53 -> 10.49, G = 32
// 16.03 -> 11.89; N = 8192, M = 32: 17.44 -> 10.38, G = 32 17.70 -> 11.92;
// 448 or 288 64-column blocks at G = 32: K = 4096, N = 14336, M = 32 20.1 vs
// 22.2; N = 6144, M = 48 19.2 vs 20.1); with K > 4096 the 4-wave loop loads
// them every k-step or two, and only two 16-row groups on 32-column blocks up
// to K = 8192 still win (N = 4096, K = 8192, M = 24 / 32: G = 64 17.55 /
// 18.88 -> 14.43 / 14.71, G = 32 17.97 / 19.39 -> 16.98 / 18.45; K = 11008
// a tie, K = 14336 2-14 % slower; 64-column blocks, N = 6144, K = 8192, G = 64:
// 22.6 vs 20.1).
// 13 <= M <= 16: two 8-row groups on 32-column blocks where those fit the CUs
// (N = 4096: K = 4096 7.61 -> 7.00 us, G = 64 / 32 7.64 / 8.70 -> 7.17 /
// 7.69; K = 14336 19.47 -> 18.13, up to K = 16384 at G = 128 only: G = 64
// 20.2 vs 22.8, K = 28672 the streamed tiles'; M <= 12, or more blocks, or
// 64-column blocks: slower).
struct SkinnyRows {
  int cfg, rows;   // cfg -1: all rows in one workgroup
};
SkinnyRows skinny_row_groups(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  if (M <= 12 || M > kSkinnyMaxM) return {-1, 0};
  const bool g128 = G % 128 == 0;
  const bool c2 = N % 2 == 0, c3 = N % 4 == 0;
  // M = 16 with one batch per wave on 8 or 16 waves (1024 < K <= 4096): the
  // whole 16-row tile, whose activations the kernel stages in LDS by
  // whole-line loads (measured on MI355X, K = N = 4096: two 8-row groups on
  // 32-column blocks 6.78 / 7.31 us at G = 128 / 32 against 6.31 / 6.76 on
  // 16-column blocks of all 16 rows)
  if (M == 16 && K > 1024 && K <= 4096) return {-1, 0};
  if (M <= 16)
    return c2 && (N + 31) / 32 * 2 <= cus && (K <= 4096 || (g128 && K <= 16384))
               ? SkinnyRows{2, 8}
               : SkinnyRows{-1, 0};
  const int64_t g = (M + 15) / 16;
  const int64_t wg2 = (N + 31) / 32 * g, wg3 = (N + 63) / 64 * g;
  if (K <= 4096) {
    if (c2 && wg2 <= cus) return {2, 16};
    // 64-column blocks over as many rounds as keep rounds x K within 8192
    // (4096 at G = 32 with K <= 1024, where the activations are not staged):
    // a round's workgroups are short at small K
    if (c3 && wg3 * K <= (G % 64 == 0 || K > 1024 ? 8192 : 4096) * (int64_t)cus) return {3, 16};
    return {-1, 0};
  }
  if (c2 && wg2 <= cus && K <= (g128 ? 16384 : 8192) && (g == 2 || g128)) return {2, 16};
  if (c3 && g128 && M >= 24 && wg3 <= cus && K <= 8192) return {3, 16};
  return {-1, 0};
}

// k-splits for the streamed kernel on few tiles: about 448 workgroups, at
// least 8 k-steps per split, and never more workgroups than two per CU (a
// split that spills into a second round costs its partials and a round:
// M = 256, K = 3584, N = 37888, 296 tiles: 97.3 us at 2 splits, 84.8 unsplit;
// M = 64, 148 64-row tiles: 44.2 at 4, 39.4 at 2).
int stream_split_for(int64_t tiles, int64_t K, int cus) {
  if (tiles <= 0) return 1;
  const int64_t kt = K / 64;
  int64_t s = (448 + tiles - 1) / tiles;
  if (s * tiles > 2 * (int64_t)cus) s = 2 * (int64_t)cus / tiles;
  if (s > kt / 8) s = kt / 8;
  return s < 1 ? 1 : (int)s;
}

// k-splits for streamed tiles when they are few (<= 64 tiles): the split
// whose workgroups (tiles x splits, after the kernel's rounding of splits to
// whole 4-step blocks of >= 8 steps) come closest to one per CU from below,
// where that fills 3/4 of the CUs with at least 10 64-k steps per split; 0
// where it does not.
// Found by the planner audit (bench.py --planner-audit: static plan against
// every other plan), measured on MI355X (µs) against the ~448 workgroups of
// stream_split_for, 64-row tiles: M = 64, K = N = 8192 (32 tiles) 25.4 ->
// 23.3 at 256 workgroups; M = 64, K = 14336, N = 4096 (16 tiles) 26.2 ->
// 23.7 at 224; M = 64, K = 5120, N = 15360 (60 tiles) 26.7 -> 25.5 at 240.
// Shorter splits lose: M = 64, K = N = 5120 (20 tiles) 19.7 at 200
// workgroups of 8 steps against 18.6 for 40 32-row tiles at 200 of 16
// steps (K = 11008, 16 tiles: 22.0 at 240 of 12 steps, the best plan).
// With more tiles, and for M <= 32, two per CU win (stream_split_two).
int stream_split_one_per_cu(int64_t tiles, int64_t K, int cus) {
  if (tiles <= 0 || tiles > 64) return 0;
  const int64_t smax = K / 64 / 8;
  int one = 0;
  int64_t u1 = 0;
  for (int64_t s = 1; s <= smax && s <= 64; ++s) {
    const int64_t u = tiles * stream_splits((int)K, (int)s);
    if (u <= cus && u > u1) u1 = u, one = (int)s;
  }
  if (!one || u1 * 4 < 3 * (int64_t)cus) return 0;
  const int64_t splits = stream_splits((int)K, one);
  return (K / 64 + splits - 1) / splits >= 10 ? one : 0;
}

// k-splits for the 32-row streamed tiles and for the 64-row ones past 64
// tiles: the split whose workgroups (after the kernel's rounding) come
// closest to two per CU from below, 2 % over allowed.  Against
// stream_split_for, which ignores the rounding (µs on MI355X): M = 32,
// K = 4096, N = 22016 (86 tiles) 23.5 -> 22.4 at 516 workgroups; M = 32,
// K = 8192, N = 10240 (40 tiles) 24.1 -> 22.6 at 440; M = 32, K = 4096,
// N = 28672 (112 tiles) 25.3 at 448 (224: 28.5).
int stream_split_two(int64_t tiles, int64_t K, int cus) {
  if (tiles <= 0) return 1;
  const int64_t smax = K / 64 / 8;
  int two = 1;
  int64_t u2 = 0;
  for (int64_t s = 1; s <= smax && s <= 64; ++s) {
    const int64_t u = tiles * stream_splits((int)K, (int)s);
    if (u * 100 <= 2 * (int64_t)cus * 102 && u > u2) u2 = u, two = (int)s;
  }
  return two;
}

MfmaChoice mfma_choice_rules(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  if (M <= 64) {
    if (!mfma_cfg_applicable(12, (int)M, (int)N, (int)K, (int)G)) return {2, 1};
    const int rows = M <= 32 ? 32 : 64;
    const int64_t tiles = (N + 255) / 256 * ((M + rows - 1) / rows);
    if (rows == 64) {
      // 64-row tiles one per CU, else 32-row tiles one per CU, else 64-row
      // tiles two per CU
      const int s1 = stream_split_one_per_cu(tiles, K, cus);
      if (s1) return {13, s1 > 1 ? stream_splits((int)K, s1) : 1};
      const int s32 = stream_split_one_per_cu(2 * tiles, K, cus);
      if (s32) return {12, s32 > 1 ? stream_splits((int)K, s32) : 1};
    }
    int s = stream_split_two(tiles, K, cus);
    // 32-row tiles beyond one round of two per CU (LM-head widths): split two
    // ways where that packs them into fewer full rounds (594 tiles, M = 16,
    // K = 4096 / 3584, N = 151936 / 152064: 99.1 / 87.3 -> 91.9 / 79.4 us;
    // 501 tiles, N = 128256, unsplit, are within one round; the 64-row tiles
    // of M = 64 at N = 151936 measured no faster split)
    const int64_t slots = 2 * (int64_t)cus;
    if (rows == 32 && tiles > slots && K / 64 / 2 >= 8 &&
        (2 * tiles + slots - 1) / slots < 2 * ((tiles + slots - 1) / slots))
      s = 2;
    return {M <= 32 ? 12 : 13, s > 1 ? stream_splits((int)K, s) : 1};
  }
  // 64-row tiles (cfg 13, one k-slice) split for about two workgroups per CU,
  // ahead of the 128-row tilings, where those waste rows or have few tiles:
  //   * 128 < M <= 192 with at most 160 64-row tiles: the last 128-row tile
  //     is at most half used (M = 192: a quarter of the MFMA work padding);
  //   * M <= 128, K >= 8192 with at most 40 64-row tiles (down-projections):
  //     more, shorter workgroups than the two-slice kernel's one per tile;
  // both only where the splits keep at least 10 k-steps each (K = N = 4096,
  // M = 192, 48 tiles: 8 splits of 8 steps 25.5 us against 23.3 for the
  // rule below's 4).
  // Measured on MI355X against the plans before (µs, G = 128 / 64 / 32, warm
  // weights, graph replay): M = 192, K = 4096, N = 6144 29.9 / 29.8 / 30.0 ->
  // 27.5 / 27.9 / 27.1; K = N = 5120 29.0 / 28.4 / 29.3 -> 26.0 / 25.5 / 26.7;
  // K = 13824, N = 5120 47.0 / 46.4 / 48.9 -> 41.9 / 42.4 / 43.2; K = 8192,
  // N = 10240 52.2 / 52.3 / 54.4 -> 46.6 / 46.6 / 47.6; K = 4096, N = 12288
  // 38.7 / 38.8 / 41.9 -> 38.1 / 37.6 / 38.5; M = 96 / 128, K = 11008, N =
  // 4096 27.8 / 28.9 -> 26.3 / 27.2 (G = 32: 28.7 / 29.7 -> 26.7 / 27.8);
  // K = 13824, N = 5120 33.0 / 34.4 -> 31.6 / 33.1.  Not taken: more 64-row
  // tiles (K = 5120, N = 15360, M = 192, 180 tiles: 46.9 on cfg 14 against
  // 49.3 at best; the gate+up layers).  Long rows gain most (planner audit,
  // M = 192, G = 128: K = 16384 / 28672, N = 5120 +16 / +14 %; K = 20480,
  // N = 10240 +14 %; K = 28672, N = 6144 +6 %); on 96 tiles (N = 8192) the
  // plan stays within 1 % of cfg 14 and 3-4 % behind cfg 11 split eight
  // ways at K = 28672, and 3 % behind cfg 14 at K = 8192 (42.2 vs 40.8).
  // With G % 128 != 0 (a scale / zero load every k-step or half-step, which
  // costs the two-slice kernel more) the few-tile case reaches 64 tiles up to
  // K = 16384 (planner audit, K = N = 8192, M = 96 / 128: G = 64 29.8 / 32.4
  // -> 28.8 / 31.3, G = 32 31.4 / 34.6 -> 29.9 / 32.3; at G = 128 within 2 %
  // either way, and K = 28672 on 64 tiles 12 % slower on cfg 13).
  if (M <= 256 && mfma_cfg_applicable(13, (int)M, (int)N, (int)K, (int)G)) {
    const int64_t t13 = (N + 255) / 256 * ((M + 63) / 64);
    const bool half_tile = M > 128 && M <= 192 && t13 <= 160;
    const bool few = M <= 128 && K >= 8192 &&
                     (t13 <= 40 || (G % 128 != 0 && t13 <= 64 && K <= 16384));
    if (half_tile || few) {
      const int s = stream_split_two(t13, K, cus);
      const int ns = s > 1 ? stream_splits((int)K, s) : 1;
      if ((K / 64 + ns - 1) / ns >= 10) return {13, ns};
    }
  }
  const bool c11 = mfma_cfg_applicable(11, (int)M, (int)N, (int)K, (int)G);
  const bool c7 = mfma_cfg_applicable(7, (int)M, (int)N, (int)K, (int)G);
  const int64_t t6 = ((N + 255) / 256) * ((M + 127) / 128);
  // 128 x 256 tiles that fit one per CU: cfg 14 (the cfg 11 kernel with two
  // k-slices per workgroup, one workgroup per CU), split along K for about a
  // workgroup per CU with at least 4 steps per slice, instead of cfg 11 split
  // for two per CU (whose fp32 partials and reduction cost more).  Any G:
  // with G % 64 != 0 (a scale / zero load per half-step) the kernel spills a
  // few registers but still wins on most shapes (planner audit, G = 32, µs:
  // M = 512, K = 4096, N = 12288 68.6 -> 63.5; N = 28672, M = 256 73.2 ->
  // 64.8; C5 M = 256, K = 8192, N = 28672 134.9 -> 123.5; M = 512, K = 5120,
  // N = 15360 90.4 -> 80.6), except with 80..128 tiles (below).
  // Measured on MI355X against the plans before it (µs): C4 M = 512 81.2 ->
  // 67.5; M = 384, K = 4096, N = 14336 67.0 -> 60.0; C5 M = 256, K = 8192,
  // N = 28672 137.5 -> 126.3 (G = 64: 135.0 -> 127.6); C5 M = 256, K = 28672,
  // N = 8192 132.3 -> 128.8 (4 splits); M = 128, K = 4096, N = 14336 34.9 ->
  // 32.0 (4 splits); M = 512, K = N = 4096 38.8 -> 36.0; M = 256, K = 14336,
  // N = 4096 48.5 -> 46.2 (8 splits); ties at M = 128 / 256, K = N = 4096.
  // More tiles than CUs (M = 1024, N = 14336: 131.0 vs 119.4) keep cfg 11.
  // Unsplit it needs its tiles to fill 7/10 of the CUs, or K <= 4096: with
  // 160 tiles for 256 CUs (one workgroup each, the rest idle) and longer K,
  // cfg 11 split three ways for about two workgroups per CU wins instead
  // (measured on MI355X, µs: M = 1024, K = 13824, N = 5120 174.9 -> 138.9;
  // M = 512, K = 8192, N = 10240 108.1 -> 92.1; M = 1024, K = N = 5120 70.7 ->
  // 66.6), not at K = 4096 (172 tiles, M = 256, N = 22016: 59.9 unsplit
  // against 64.8 split two ways); 192 tiles, M = 512, K = 4096, N = 12288:
  // cfg 14 within 2 %.  Split two ways or more it keeps winning (86 tiles,
  // M = 128, K = 4096, N = 22016).
  const int64_t s14 = t6 > 0 ? (cus / t6 < K / 512 ? cus / t6 : K / 512) : 1;
  const bool fills = s14 > 1 || t6 * 10 >= 7 * (int64_t)cus || K <= 4096;
  if (c11 && t6 <= cus && fills) {
    int64_t s = s14;
    if (s < 1) s = 1;
    // 64 < M <= 256 on small layers: the 64-row streamed tiles (cfg 13, one
    // k-slice) instead, where the two-slice split would leave each slice at
    // most 4 k-steps (K / s <= 512; then split for about a workgroup per CU,
    // >= 8 k-steps each), or, with K <= 2048, unsplit where their tiles give
    // half the CUs one each (no partials, no reduction pass).  Measured on
    // MI355X against cfg 14's plan (µs, G = 128): K = N = 4096, M = 96 / 128 /
    // 192 / 256: 22.3 / 24.2 / 28.8 / 29.2 -> 19.4 / 21.3 / 24.6 / 26.4;
    // K = 2048, N = 4096, M = 96 / 128 / 192: 18.0 / 19.7 / 22.2 -> 14.5 /
    // 16.0 / 18.8; K = 2048, N = 16384, M = 96 / 128 / 192 / 256: 25.9 / 27.4
    // / 30.9 / 33.9 -> 24.7 / 26.5 / 25.7 / 26.0.  Longer slices keep cfg 14
    // (K = 4096, N = 14336, M = 96 / 128: 28.0 / 30.3 vs 28.3 / 30.2 at best;
    // K = 14336, N = 4096 and K = N = 8192 ties or slower; unsplit at K = 4096
    // 47 us at every M).
    // M <= 128 with 86..128 64-row tiles: those, split for about two
    // workgroups per CU (µs: M = 128, K = 5120, N = 15360, 120 tiles: 34.5 at
    // 480 workgroups against 37.8 for cfg 14 at 240; K = 4096, N = 12288, 96
    // tiles: 29.0 against 29.7).  Outside that range cfg 14 is as fast or
    // faster (K = 5120, N = 27648, 216 tiles; K = 8192, N = 10240, 80 tiles);
    // K <= 2048 keeps the unsplit 64-row tiles below.
    if (M <= 128 && K > 2048) {
      const int64_t t13 = (N + 255) / 256 * ((M + 63) / 64);
      if (t13 >= 86 && t13 <= 128) {
        const int s13 = stream_split_two(t13, K, cus);
        return {13, s13 > 1 ? stream_splits((int)K, s13) : 1};
      }
    }
    if (M <= 256 && s > 1) {
      const int64_t t13 = (N + 255) / 256 * ((M + 63) / 64);
      if (K <= 2048 && 2 * t13 >= cus) return {13, 1};
      // from K = 4096 at least 10 k-steps per split (M = 128, K = N = 4096,
      // 32 tiles: 20.0 us at 6 splits of 11 steps against 20.7 at 8 of 8
      // steps); shorter K keeps 8 (measured at K = 4096 only)
      if (K / s <= 512) {
        int64_t s13 = cus / t13;
        if (s13 > K / (K >= 4096 ? 640 : 512)) s13 = K / (K >= 4096 ? 640 : 512);
        if (s13 < 1) s13 = 1;
        return {13, s13 > 1 ? stream_splits((int)K, (int)s13) : 1};
      }
    }
    // Long rows (K >= 16384) on fewer tiles than CUs: cfg 11 (two workgroups
    // resident per CU) split along K, whose partials and reduction are small
    // beside rows that long -- from 86 tiles the most of eight, four or two
    // splits that makes at most three workgroups per CU, and from K = 24576
    // with more than 64 tiles split for about two workgroups per CU.  Measured on
    // MI355X (planner audit, µs, against cfg 14's plan), N = 8192: K = 28672,
    // M = 384 (96 tiles) 177.1 at eight splits (185.2 at four); M = 512 (128
    // tiles) 218.8 -> 209.8; M = 768 (192 tiles), K = 28672 / 20480 / 16384
    // 365.0 / 272.0 / 207.8 -> 330.1 / 241.2 / 199.3; N = 10240, K = 20480,
    // M = 768 (240 tiles) 285.4 at two splits (300.6 at four); N = 5120,
    // K = 16384, M = 768 (120 tiles) 124.2, best; K = 28672: 72 tiles (N =
    // 6144, M = 384) 145.7 -> 138.4 (6 splits), 80 (N = 5120, M = 512) 144.0
    // (6), best; 64 tiles (N = 8192, M = 256) keep cfg 14 at four splits, a
    // tie (116.4 against 115.3 at eight) with half the partials, and so do
    // shorter rows (K = 16384, 80 tiles: 91.8 with three splits, best; K =
    // 11008, 128 tiles, M = 1024, N = 4096: 92.3, best).
    if (K >= 16384 && t6 < cus) {
      if (t6 >= 86) {
        const int64_t w3 = 3 * (int64_t)cus;
        return {11, stream_splits((int)K, t6 * 8 <= w3 ? 8 : t6 * 4 <= w3 ? 4 : 2)};
      }
      if (K >= 24576 && (t6 > 64 || (G % 64 != 0 && t6 >= 60)))
        return {11, stream_splits((int)K, stream_split_two(t6, K, cus))};
    }
    // G % 64 != 0 (a scale / zero load per half-step, where the two-slice
    // kernel spills a few registers) with 80..128 tiles past K = 4096: cfg 11
    // split for about two workgroups per CU (measured on MI355X, G = 32, µs:
    // M = 512, K = N = 5120 (80 tiles) 46.3 -> 43.8; M = 1024, K = 14336,
    // N = 4096 (128 tiles) 123.8 -> 118.5; K = 13824, N = 5120, M = 512 82.9
    // -> 81.3)
    if (G % 64 != 0 && t6 >= 80 && t6 <= 128 && K > 4096)
      return {11, stream_splits((int)K, stream_split_two(t6, K, cus))};
    return {14, s > 1 ? stream_splits((int)K, (int)s, 2) : 1};
  }
  // M >= 1024 with more tiles than CUs but fewer than two per CU: split K
  // three ways where that packs the tiles into two full rounds of two
  // workgroups per CU instead of one partly filled round (320 tiles: M = 1024,
  // K = 8192, N = 10240 188.6 -> 179.6 us on MI355X); else unsplit.
  if (M >= 1024 && c11 && t6 > cus && 3 * t6 <= 4 * (int64_t)cus && K / 64 >= 24)
    return {11, stream_splits((int)K, 3)};
  if (M >= 1024 && (c11 || c7) && t6 > cus) return {c11 ? 11 : 7, 1};
  // cfg 11 on fewer than ~448 tiles: split K for about two workgroups per CU
  // (measured on MI355X: M = 128, K = 8192, N = 28672: 77.7 us at 4 splits vs
  // 90.2 at 3; M = 256: 133.2 at 2 vs 149.8 unsplit; M = 256, K = 28672, N =
  // 8192: 137.9 at 7 vs 146.8 at 4; M = 512, K = 4096, N = 14336: 80.8 at 2 vs
  // 82.7)
  if (c11 && t6 < 448) {
    const int s = stream_split_for(t6, K, cus);
    if (s >= 2) return {11, stream_splits((int)K, s)};
  }
  if (2 * t6 >= cus) {
    if (c11) return {11, 1};
    if (mfma_cfg_applicable(6, (int)M, (int)N, (int)K, (int)G)) return {6, 1};
  }
  if (c7) {
    const int64_t kt = K / 64;
    int64_t s = (cus + t6 - 1) / t6;
    if (s > kt / 8) s = kt / 8;
    if (s >= 2) return {7, occ2_splits((int)K, (int)s)};
  }
  const int64_t t2 = ((N + 511) / 512) * ((M + 31) / 32);
  if (2 * t6 < cus && t2 > t6) return {2, 1};
  return {1, 1};
}

// Work of the busiest CU under a streamed plan, in row x k-step units: the
// workgroups each CU receives (tiles x splits over the CUs, rounded up) x
// rows per tile x k-steps per split.
int64_t stream_cu_load(int64_t tiles, int rows, int split, int64_t K, int cus) {
  const int64_t ks = K / 64;
  return (tiles * split + cus - 1) / cus * rows * ((ks + split - 1) / split);
}

// 256 < M <= 512, K <= 12288: the 64-row tiles (cfg 13, one k-slice) split
// for about two workgroups per CU instead of the 128-row plan where the
// busiest CU's work falls to 5/6 or less (the last 128-row tile partly
// padding, or 128-row tiles past one round), or stays level on splits of at
// most 20 k-steps (where the two-slice kernel's short slices cost more); at
// most two workgroups per CU, at least 10 k-steps per split.
// Measured on MI355X (planner audit and probe, G = 128, µs, 128-row plan ->
// 64-row plan): M = 288 / 320, K = 4096: N = 12288 57.1 / 57.2 -> 47.4 /
// 47.5 (work 1/2); N = 11008 56.6 / 56.6 -> 45.4 / 46.5 (1/2); N = 22016
// (258 128-row tiles) 95.5 / 96.3 -> 71.0 / 72.1 (1/2); N = 6144 35.1 / 35.8
// -> 29.9 / 30.9 (3/4); N = 4096 29.8 / 30.8 -> 27.5 / 28.1 (2/3); K = N =
// 5120 36.3 / 37.4 -> 31.1 / 31.9 (4/5); K = N = 8192 63.6 / 64.0 -> 59.5 /
// 60.9 (2/3); K = 11008, N = 4096 48.0 / 49.6 -> 46.0 / 47.9 (5/6; G = 32
// 49.5 / 51.2 -> 47.0 / 48.2); level work, 16-20 k-steps: M = 384 / 448 /
// 512, K = N = 4096 32.9 / 34.3 / 34.4 -> 30.2 / 31.4 / 32.6; M = 384,
// K = N = 5120 38.0 -> 34.6.  Kept: level work on longer splits (M = 320, K = 8192, N = 10240,
// 12-14 % slower; K = 5120, N = 15360), more than two 64-row tiles per CU
// (the 8B / 13B / 70B gate+up layers, 6-11 % slower), and K >= 13824 (5/6 of
// the work, 1-3 % slower).
MfmaChoice mfma_choice(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  const MfmaChoice c = mfma_choice_rules(M, N, K, G, cus);
  if (M <= 256 || M > 512 || K > 12288 || (c.cfg != 11 && c.cfg != 14) ||
      !mfma_cfg_applicable(13, (int)M, (int)N, (int)K, (int)G))
    return c;
  const int64_t t13 = (N + 255) / 256 * ((M + 63) / 64);
  const int64_t t6 = (N + 255) / 256 * ((M + 127) / 128);
  const int s = stream_split_two(t13, K, cus);
  const int ns = s > 1 ? stream_splits((int)K, s) : 1;
  const int64_t steps = (K / 64 + ns - 1) / ns;
  if (t13 * ns > 2 * (int64_t)cus || steps < 10) return c;
  const int64_t l13 = stream_cu_load(t13, 64, ns, K, cus);
  const int64_t l6 = stream_cu_load(t6, 128, c.split, K, cus);
  if (6 * l13 <= 5 * l6 || (l13 <= l6 && steps <= 20)) return {13, ns};
  return c;
}

// Measured decode plans (M <= 2, 256 CUs): per group-size class (G % 128 ==
// 0, G % 64 == 0, other G % 32 == 0) and (M, K, N) of a grid, the fastest
// GEMV or skinny plan, timed on MI355X with cold weights by bench.py
// --decode-scan (--audit-g for the class) and written into decode_table.inc
// by bench.py --decode-table.  A shape inside its class's grid takes the plan
// of the nearest grid point in (log2 K, log2 N).  The rules below cover
// everything else (other M, other CU counts, shapes outside the grid).
// Measured against those rules on the same grid: 71 of 168 G = 128 shapes
// had been more than 3 % slower than the grid's best (up to 61 %: M = 2,
// K = 28672, N = 14336, 66.0 against 41.1 us on 64-column MFMA-dot blocks).
struct DecodeEntry {
  int G, M, K, N, kernel, cfg, cols, rows, split, us100, rule_us100;
};
const DecodeEntry kDecodeTable[] = {
#include "decode_table.inc"
    {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}};

int decode_gclass(int64_t G) { return G % 128 == 0 ? 128 : G % 64 == 0 ? 64 : 32; }

// One (group class, M) slice of the table as a grid: its distinct K and N
// (ascending, with their log2) and the entry at each grid point.  Built once;
// a lookup is then two short nearest-value scans instead of a log2 per entry.
struct DecodeGrid {
  int gclass = 0, M = 0;
  std::vector<int64_t> ks, ns;
  std::vector<double> lk, ln;
  std::vector<const DecodeEntry*> at;   // [ik * ns.size() + in]
};

const std::vector<DecodeGrid>& decode_grids() {
  static const std::vector<DecodeGrid> grids = [] {
    std::vector<DecodeGrid> out;
    for (int gc : {128, 64, 32})
      for (int m : {1, 2}) {
        DecodeGrid g;
        g.gclass = gc;
        g.M = m;
        for (const DecodeEntry* e = kDecodeTable; e->M; ++e)
          if (e->G == gc && e->M == m) {
            g.ks.push_back(e->K);
            g.ns.push_back(e->N);
          }
        if (g.ks.empty()) continue;
        for (auto* v : {&g.ks, &g.ns}) {
          std::sort(v->begin(), v->end());
          v->erase(std::unique(v->begin(), v->end()), v->end());
        }
        for (int64_t k : g.ks) g.lk.push_back(std::log2((double)k));
        for (int64_t n : g.ns) g.ln.push_back(std::log2((double)n));
        g.at.assign(g.ks.size() * g.ns.size(), nullptr);
        for (const DecodeEntry* e = kDecodeTable; e->M; ++e) {
          if (e->G != gc || e->M != m) continue;
          const size_t ik = std::lower_bound(g.ks.begin(), g.ks.end(), (int64_t)e->K) - g.ks.begin();
          const size_t in = std::lower_bound(g.ns.begin(), g.ns.end(), (int64_t)e->N) - g.ns.begin();
          g.at[ik * g.ns.size() + in] = e;
        }
        out.push_back(std::move(g));
      }
    return out;
  }();
  return grids;
}

// Index of the value nearest to x (first of equals), by |log2 distance|.
size_t nearest_log(const std::vector<double>& lv, double x) {
  size_t best = 0;
  for (size_t i = 1; i < lv.size(); ++i)
    if (std::fabs(lv[i] - x) < std::fabs(lv[best] - x)) best = i;
  return best;
}

const DecodeEntry* decode_table_entry(int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
  if (M < 1 || M > 2 || G % 32 != 0 || cus != 256) return nullptr;
  const int gc = decode_gclass(G);
  for (const DecodeGrid& g : decode_grids()) {
    if (g.gclass != gc || g.M != M) continue;
    if (K < g.ks.front() || K > g.ks.back() || N < g.ns.front() || N > g.ns.back())
      return nullptr;
    const size_t ik = nearest_log(g.lk, std::log2((double)K));
    const size_t in = nearest_log(g.ln, std::log2((double)N));
    return g.at[ik * g.ns.size() + in];
  }
  return nullptr;
}

size_t mfma_workspace_bytes(int64_t M, int64_t N, int64_t K, int split) {
  return occ2_workspace_bytes((int)M, (int)N, (int)K, split);
}

// G % 64 != 0 (a scale / zero load every 32 k, which the skinny kernel's
// 4-wave loop pays in every k-step), M = 3..4, long rows on 3072..4096
// columns: the GEMV on 64-column blocks split four ways (256 workgroups)
// instead of the skinny kernel.  Measured on MI355X, G = 32, N = 4096, µs,
// skinny -> GEMV: M = 3, K = 11008 / 14336 / 16384 / 20480 / 28672 15.3 /
// 17.9 / 20.2 / 24.2 / 32.3 -> 13.4 / 16.3 / 16.6 / 18.8 / 27.0; M = 4 15.5 /
// 18.4 / 20.4 / 24.6 / 32.3 -> 14.5 / 17.6 / 17.8 / 21.2 / 26.9.  Not at
// K = 8192 (a tie at M = 3, 3.6 % slower at M = 4), N = 5120 (mixed), M >= 5
// or with larger groups (the skinny kernel stays fastest).
bool small_m_long_k_gemv(int64_t M, int64_t N, int64_t K, int64_t G) {
  return G % 64 != 0 && M >= 3 && M <= 4 && K >= 11008 && N >= 3072 && N <= 4096 && N % 4 == 0;
}

int make_plan(int64_t M, int64_t N, int64_t K, int64_t G, int32_t kernel, int32_t split,
              w4a16_plan* p) {
  const int cus = device_cu_count();
  *p = w4a16_plan{};
  // Empty shapes (forced families included) plan the SIMT kernel: nothing is
  // launched for M = 0 or N = 0, and K = 0 writes y = 0 with it.  (The tile
  // and block counts of the other families would be zero, and their split
  // rules divide by them.)
  if (kernel != W4A16_KERNEL_AUTO && kernel != W4A16_KERNEL_GEMV && kernel != W4A16_KERNEL_MFMA &&
      kernel != W4A16_KERNEL_SIMT && kernel != W4A16_KERNEL_SKINNY)
    return W4A16_ERR_BAD_PLAN;
  if (M == 0 || N == 0 || K == 0) kernel = W4A16_KERNEL_SIMT;
  if (kernel == W4A16_KERNEL_AUTO && fits(M, N, K, G)) {
    if (const DecodeEntry* e = decode_table_entry(M, N, K, G, cus)) {
      if (e->kernel == W4A16_KERNEL_GEMV && gemv_applicable(M, N, G) &&
          gemv_cfg_valid(e->cfg, (int)M, e->cols) && gemv_cols_valid(e->cols)) {
        int S = e->split < K / 8 ? e->split : (int)(K / 8);
        if (S > 1) {
          const int64_t KP = K / 8, rows = (KP + S - 1) / S;
          S = (int)((KP + rows - 1) / rows);
        }
        p->kernel = W4A16_KERNEL_GEMV;
        p->split_k = S < 1 ? 1 : S;
        p->tile_cfg = e->cfg;
        p->tile_m = 0;
        p->tile_n = e->cols;
        p->grid_x = ((N + e->cols - 1) / e->cols) * p->split_k;
        p->grid_y = 1;
        p->workspace_bytes = (int64_t)gemv_workspace_bytes((int)M, (int)N, (int)K, p->split_k);
        return W4A16_OK;
      }
      if (e->kernel == W4A16_KERNEL_SKINNY && skinny_applicable(M, G) &&
          skinny_plan_valid(e->cfg, (int)M, (int)N, e->rows)) {
        p->kernel = W4A16_KERNEL_SKINNY;
        p->split_k = 1;
        p->tile_cfg = e->cfg;
        p->tile_m = e->rows;
        p->tile_n = e->cfg == 3 ? 64 : e->cfg == 2 ? 32 : 16;
        p->grid_x = (N + p->tile_n - 1) / p->tile_n * ((M + p->tile_m - 1) / p->tile_m);
        p->grid_y = 1;
        return W4A16_OK;
      }
    }
  }
  if (kernel == W4A16_KERNEL_AUTO) {
    if (!fits(M, N, K, G))
      kernel = W4A16_KERNEL_SIMT;
    else if (skinny_applicable(M, G) && skinny_row_groups(M, N, K, G, cus).cfg >= 0)
      kernel = W4A16_KERNEL_SKINNY;
    else if (gemv_applicable(M, N, G) && small_m_long_k_gemv(M, N, K, G))
      kernel = W4A16_KERNEL_GEMV;
    else if (small_m_takes_stream(M, N, K, G))
      kernel = skinny_applicable(M, G) && (skinny_quad(M, N, K, G, cus) ||
                                           skinny_wide_beats_stream(M, N, K, G, cus))
                   ? W4A16_KERNEL_SKINNY
                   : W4A16_KERNEL_MFMA;
    else if (gemv_applicable(M, N, G) && !decode_takes_skinny(M, N, K, G, cus))
      kernel = W4A16_KERNEL_GEMV;
    else if (M <= kSkinnyMaxM && skinny_applicable(M, G))
      kernel = W4A16_KERNEL_SKINNY;
    else if (mfma_applicable(N, G))
      kernel = W4A16_KERNEL_MFMA;
    else
      kernel = W4A16_KERNEL_SIMT;
  }
  p->kernel = kernel;
  p->split_k = 1;
  switch (kernel) {
    case W4A16_KERNEL_GEMV: {
      if (!gemv_applicable(M, N, G)) return W4A16_ERR_BAD_PLAN;
      const int mfma_split = split > 0 ? 0 : gemv_mfma_split(M, N, K, cus);
      const bool g32 = split <= 0 && small_m_long_k_gemv(M, N, K, G);
      const int cols = mfma_split ? 64 : g32 ? 64 : gemv_cols_auto(M, N, K, cus);
      int S = split > 0                                   ? split
              : g32                                       ? 4
              : mfma_split                                ? mfma_split
              : cols == 64 && gemv_band64(M, N, K, cus)   ? 1
              : cols == 32 && gemv_band32(N, cus)         ? 1
              : cols == 128 && M <= 2                     ? 1
                                                          : gemv_split_auto(N, K, cols, cus);
      const int64_t KP = K / 8;
      if (KP == 0) S = 1;
      if (S > 1) {
        if (S > KP) S = (int)KP;
        const int64_t rows = (KP + S - 1) / S;
        S = (int)((KP + rows - 1) / rows);
      }
      p->split_k = S;
      p->tile_cfg = mfma_split ? kGemvDefaultConfig + 6 : gemv_waves_cfg(M, K, S, cols);
      p->tile_m = 0;
      p->tile_n = cols;
      p->grid_x = ((N + cols - 1) / cols) * S;
      p->grid_y = 1;
      p->workspace_bytes = (int64_t)gemv_workspace_bytes((int)M, (int)N, (int)K, S);
      return W4A16_OK;
    }
    case W4A16_KERNEL_MFMA: {
      if (!mfma_applicable(N, G)) return W4A16_ERR_BAD_PLAN;
      MfmaChoice c = mfma_choice(M, N, K, G, cus);
      if (split > 0) {   // a forced split runs on the streamed kernel (cfg 7 where K % 256 != 0)
        const bool c11 = mfma_cfg_applicable(11, (int)M, (int)N, (int)K, (int)G);
        c.cfg = split > 1 ? (c.cfg >= 11 ? c.cfg : (c11 ? 11 : 7)) : c.cfg;
        // two k-slices split K in 8-step units: where that makes fewer splits
        // than asked for, the one-slice kernel's 4-step units honour the request
        if (split > 1 && c.cfg == 14 && stream_splits((int)K, split, 2) < stream_splits((int)K, split, 1))
          c.cfg = 11;
        c.split = split > 1 ? (c11 ? stream_splits((int)K, split, c.cfg == 14 ? 2 : 1)
                                   : occ2_splits((int)K, split))
                            : 1;
        if (c.split > 1 && !mfma_cfg_applicable(c.cfg, (int)M, (int)N, (int)K, (int)G))
          return W4A16_ERR_BAD_PLAN;
      }
      const MfmaTile t = mfma_tile(c.cfg);
      p->tile_cfg = c.cfg;
      p->split_k = c.split;
      p->tile_m = t.bm;
      p->tile_n = t.bn;
      p->grid_x = ((N + t.bn - 1) / t.bn) * ((M + t.bm - 1) / t.bm) * c.split;
      p->grid_y = 1;
      p->workspace_bytes = (int64_t)mfma_workspace_bytes(M, N, K, c.split);
      return W4A16_OK;
    }
    case W4A16_KERNEL_SKINNY: {
      if (!skinny_applicable(M, G)) return W4A16_ERR_BAD_PLAN;
      const SkinnyRows rg = skinny_row_groups(M, N, K, G, cus);
      p->tile_m = rg.cfg >= 0 ? rg.rows : (int32_t)((M + 15) / 16 * 16);
      p->tile_n = rg.cfg >= 0           ? (rg.cfg == 3 ? 64 : 32)
                  : skinny_quad(M, N, K, G, cus) ? 64
                  : skinny_wide(M, N, cus)    ? 32
                                              : 16;
      p->grid_x = (N + p->tile_n - 1) / p->tile_n * ((M + p->tile_m - 1) / p->tile_m);
      p->grid_y = 1;
      // 64- or 32-column blocks where they apply (cfg 3 / 2), else 16-column
      // blocks (cfg 0); the kernel's wave count follows K.  (An 8-wave form
      // of the two-batch loop on 16-column blocks, once cfg 1, was nowhere
      // faster -- measured on MI355X, 4 vs 8 waves: M = 3 / 8 / 16, K = 4096,
      // N = 6144: 8.9 / 10.0 / 12.3 vs 9.3 / 10.5 / 13.0 us; M = 8 / 16,
      // K = 14336, N = 4096: 15.4 / 19.3 vs 16.2 / 19.9; M = 32, K = N = 4096:
      // 11.5 vs 12.1 -- and was retired.)
      p->tile_cfg = p->tile_n == 64 ? 3 : p->tile_n == 32 ? 2 : 0;
      return W4A16_OK;
    }
    case W4A16_KERNEL_SIMT:
      p->tile_m = 4;
      p->tile_n = 64;
      p->grid_x = (N + 63) / 64;
      p->grid_y = (M + 3) / 4;
      return W4A16_OK;
    default:
      return W4A16_ERR_BAD_PLAN;
  }
}

int to_status(hipError_t e) { return e == hipSuccess ? W4A16_OK : (int)e; }

// Row strides: ldx >= K, ldy >= N, both int32, and the strided extents
// addressable like the dense ones.
int check_strides(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy) {
  if (ldx < K || ldy < N || ldx > INT32_MAX || ldy > INT32_MAX) return W4A16_ERR_BAD_SHAPE;
  if (M > 0 && ((uint64_t)(M - 1) * (uint64_t)ldx > (1ull << 46) ||
                (uint64_t)(M - 1) * (uint64_t)ldy > (1ull << 46)))
    return W4A16_ERR_BAD_SHAPE;
  return W4A16_OK;
}

// What the vector kernels need of the strides: 16-byte x rows (16-byte loads)
// and x within one buffer resource (< 2 GiB); kernels that store 4-column
// quads of y (the MFMA family and the split-K reduction) also 8-byte y rows.
bool strides_vec_ok(const GemmArgs& a, int kernel, int split) {
  const bool quad_stores = kernel == W4A16_KERNEL_MFMA || split > 1;
  return a.ldx % 8 == 0 && (!quad_stores || a.ldy % 4 == 0) &&
         x_extent_bytes(a) < (1ull << 31);
}

int run_planned(const w4a16_plan* p, const void* x, int64_t ldx, const int32_t* qw,
                const void* sc, const void* zr, const void* bias, void* y, int64_t ldy,
                int64_t M, int64_t N, int64_t K, int64_t G, void* ws, size_t ws_bytes,
                void* stream) {
  if (!p) return W4A16_ERR_NULL_POINTER;
  if (int st = check_gemm_shape(M, N, K, G)) return st;
  if (int st = check_strides(M, N, K, ldx, ldy)) return st;
  if (M == 0 || N == 0) return W4A16_OK;
  if (!y || (K > 0 && (!x || !qw || !sc || !zr))) return W4A16_ERR_NULL_POINTER;
  if (p->flags & ~W4A16_PLAN_ANY_ZEROS) return W4A16_ERR_BAD_PLAN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemmArgs a{x, qw, sc, zr, bias, y, (int)M, (int)N, (int)K, (int)G, (int)ldx, (int)ldy,
             (p->flags & W4A16_PLAN_ANY_ZEROS) != 0};
  // K = 0: Y = 0 (+ bias).  A kernel rather than a memset, so that the call
  // can be captured into a HIP graph; the SIMT kernel reads no operand then.
  if (K == 0) return to_status(launch_simt(a, s));
  if (p->kernel != W4A16_KERNEL_SIMT && !strides_vec_ok(a, p->kernel, p->split_k))
    return W4A16_ERR_BAD_PLAN;
  switch (p->kernel) {
    case W4A16_KERNEL_GEMV: {
      if (!gemv_applicable(M, N, G) || !fits(M, N, K, G) || p->split_k < 1 ||
          p->split_k > K / 8 || !gemv_cols_valid(p->tile_n) ||
          !gemv_cfg_valid(p->tile_cfg, (int)M, p->tile_n))
        return W4A16_ERR_BAD_PLAN;
      const int64_t nblk = (N + p->tile_n - 1) / p->tile_n;
      if (nblk * p->split_k > INT32_MAX) return W4A16_ERR_BAD_PLAN;
      if (!aligned(x, 16) || !aligned(qw, 16) || !aligned(sc, 8) || !aligned(zr, 8) ||
          (p->split_k > 1 && (!aligned(y, 8) || (bias && !aligned(bias, 8)))))
        return W4A16_ERR_BAD_PLAN;
      const size_t need = gemv_workspace_bytes((int)M, (int)N, (int)K, p->split_k);
      if (need > 0 && (!ws || ws_bytes < need || !aligned(ws, 256))) return W4A16_ERR_WORKSPACE;
      return to_status(launch_gemv(a, p->tile_n, p->tile_cfg, p->split_k, ws, s));
    }
    case W4A16_KERNEL_MFMA: {
      if (!mfma_applicable(N, G) || !fits(M, N, K, G) ||
          !mfma_cfg_applicable(p->tile_cfg, (int)M, (int)N, (int)K, (int)G) || p->split_k < 1 ||
          (p->split_k > 1 && !mfma_cfg_splits(p->tile_cfg)))
        return W4A16_ERR_BAD_PLAN;
      if (!aligned(x, 16) || !aligned(qw, 16) || !aligned(sc, 8) || !aligned(zr, 8) ||
          !aligned(y, 8) || (bias && !aligned(bias, 8)))
        return W4A16_ERR_BAD_PLAN;
      float* part = nullptr;
      const size_t need = mfma_workspace_bytes(M, N, K, p->split_k);
      if (need > 0) {
        if (!ws || ws_bytes < need || !aligned(ws, 256)) return W4A16_ERR_WORKSPACE;
        part = static_cast<float*>(ws);
      }
      return to_status(launch_mfma(a, p->tile_cfg, p->split_k, part, s));
    }
    case W4A16_KERNEL_SKINNY: {
      const int c = p->tile_cfg;
      if (!skinny_applicable(M, G) || !fits(M, N, K, G) ||
          !skinny_plan_valid(c, (int)M, (int)N, p->tile_m))
        return W4A16_ERR_BAD_PLAN;
      // each lane loads 1, 2 or 4 adjacent columns' words, scales and zeros
      // in one load: 4 / 8 / 16-byte weights, 2 / 4 / 8-byte scales and zeros
      const uintptr_t cols = c == 3 ? 4 : c == 2 ? 2 : 1;
      if (!aligned(x, 16) || !aligned(qw, 4 * cols) || !aligned(sc, 2 * cols) ||
          !aligned(zr, 2 * cols))
        return W4A16_ERR_BAD_PLAN;
      return to_status(launch_skinny(a, c, p->tile_m, s));
    }
    case W4A16_KERNEL_SIMT:
      return to_status(launch_simt(a, s));
    default:
      return W4A16_ERR_BAD_PLAN;
  }
}

// Automatic plan, falling back to the SIMT kernel when the pointers or row
// strides do not meet the vector kernels' alignment.  Shape and strides must
// have been checked.
int auto_plan(const void* x, int64_t ldx, const int32_t* qw, const void* sc, const void* zr,
              const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t G,
              w4a16_plan* p) {
  if (int st = make_plan(M, N, K, G, W4A16_KERNEL_AUTO, 0, p)) return st;
  const GemmArgs a{x, qw, sc, zr, bias, y, (int)M, (int)N, (int)K, (int)G, (int)ldx, (int)ldy};
  const bool vec_aligned = aligned(x, 16) && aligned(qw, 16) && aligned(sc, 8) &&
                           aligned(zr, 8) && aligned(y, 8) && (!bias || aligned(bias, 8)) &&
                           strides_vec_ok(a, p->kernel, p->split_k);
  if (p->kernel != W4A16_KERNEL_SIMT && !vec_aligned)
    return make_plan(M, N, K, G, W4A16_KERNEL_SIMT, 0, p);
  return W4A16_OK;
}

int run_auto(const void* x, int64_t ldx, const int32_t* qw, const void* sc, const void* zr,
             const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t G,
             void* ws, size_t ws_bytes, void* stream) {
  if (int st = check_gemm_shape(M, N, K, G)) return st;
  if (int st = check_strides(M, N, K, ldx, ldy)) return st;
  w4a16_plan p;
  if (int st = auto_plan(x, ldx, qw, sc, zr, bias, y, ldy, M, N, K, G, &p)) return st;
  return run_planned(&p, x, ldx, qw, sc, zr, bias, y, ldy, M, N, K, G, ws, ws_bytes, stream);
}

// Split-K partial bytes a plan's kernels write (what run_planned requires of
// the workspace).
size_t plan_scratch_bytes(const w4a16_plan& p, int64_t M, int64_t N, int64_t K) {
  if (p.split_k <= 1) return 0;
  if (p.kernel == W4A16_KERNEL_GEMV) return gemv_workspace_bytes((int)M, (int)N, (int)K, p.split_k);
  if (p.kernel == W4A16_KERNEL_MFMA) return mfma_workspace_bytes(M, N, K, p.split_k);
  return 0;
}

// ---- scratch of the allocation-free entry point ---------------------------
// The split-K partials of w4a16_gemm_f16_noalloc live in this file-scope
// device array: every GPU the library runs on holds its own copy until the
// process ends.  In host code the name is only a stand-in for the symbol;
// the array's device address on the current device comes from
// hipGetSymbolAddress (scratch_on_device), and only that address is passed
// to kernels.
static __device__ __align__(256) unsigned char scratch[W4A16_NOALLOC_SCRATCH_BYTES];

std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, resolved once per device
// (with that device current) and kept.
int scratch_on_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return W4A16_ERR_NO_DEVICE;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return e != hipSuccess ? (int)e : W4A16_ERR_NO_DEVICE;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return W4A16_OK;
}

}  // namespace

// sha256 of the sources this library was built from (set by the build).
#ifndef W4A16_SOURCE_HASH
#define W4A16_SOURCE_HASH "unknown"
#endif

extern "C" {

int w4a16_abi_version(void) { return W4A16_ABI_VERSION; }

const char* w4a16_build_id(void) { return W4A16_SOURCE_HASH; }

const char* w4a16_status_string(int status) {
  switch (status) {
    case W4A16_OK: return "ok";
    case W4A16_ERR_NULL_POINTER: return "a required pointer is NULL";
    case W4A16_ERR_BAD_SHAPE: return "invalid shape (negative size, K % 8 != 0, or too large)";
    case W4A16_ERR_BAD_GROUP: return "invalid group_size (must be > 0 and divide K)";
    case W4A16_ERR_WORKSPACE: return "workspace missing, misaligned or too small";
    case W4A16_ERR_BAD_PLAN: return "plan does not fit this shape, group size or pointers";
    case W4A16_ERR_NO_DEVICE: return "no HIP device";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

int w4a16_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t group_size, int32_t kernel,
                    int32_t split_k, w4a16_plan* plan) {
  if (!plan) return W4A16_ERR_NULL_POINTER;
  if (int st = check_gemm_shape(M, N, K, group_size)) return st;
  if (kernel < 0 || kernel > W4A16_KERNEL_SKINNY || split_k < 0) return W4A16_ERR_BAD_PLAN;
  return make_plan(M, N, K, group_size, kernel, split_k, plan);
}

int w4a16_zeros_check_f16(const void* zeros, int64_t count, int32_t* flag, void* stream) {
  if (count < 0) return W4A16_ERR_BAD_SHAPE;
  if (count == 0) return W4A16_OK;
  if (!zeros || !flag) return W4A16_ERR_NULL_POINTER;
  return to_status(launch_zeros_check(zeros, count, flag, static_cast<hipStream_t>(stream)));
}

size_t w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size) {
  w4a16_plan p;
  if (check_gemm_shape(M, N, K, group_size) != W4A16_OK) return 0;
  if (make_plan(M, N, K, group_size, W4A16_KERNEL_AUTO, 0, &p) != W4A16_OK) return 0;
  return (size_t)p.workspace_bytes;
}

int w4a16_gemm_f16(const void* x, const int32_t* qweight, const void* scales, const void* zeros,
                   void* y, int64_t M, int64_t N, int64_t K, int64_t group_size,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return run_auto(x, K, qweight, scales, zeros, nullptr, y, N, M, N, K, group_size, workspace,
                  workspace_bytes, stream);
}

int w4a16_linear_f16(const void* x, const int32_t* qweight, const void* scales,
                     const void* zeros, const void* bias, void* y, int64_t M, int64_t N,
                     int64_t K, int64_t group_size, void* workspace, size_t workspace_bytes,
                     void* stream) {
  return run_auto(x, K, qweight, scales, zeros, bias, y, N, M, N, K, group_size, workspace,
                  workspace_bytes, stream);
}

int w4a16_gemm_f16_planned(const w4a16_plan* plan, const void* x, const int32_t* qweight,
                           const void* scales, const void* zeros, const void* bias, void* y,
                           int64_t M, int64_t N, int64_t K, int64_t group_size, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return run_planned(plan, x, K, qweight, scales, zeros, bias, y, N, M, N, K, group_size,
                     workspace, workspace_bytes, stream);
}

int w4a16_gemm_f16_strided(const w4a16_plan* plan, const void* x, int64_t ldx,
                           const int32_t* qweight, const void* scales, const void* zeros,
                           const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                           int64_t group_size, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (!plan)
    return run_auto(x, ldx, qweight, scales, zeros, bias, y, ldy, M, N, K, group_size, workspace,
                    workspace_bytes, stream);
  return run_planned(plan, x, ldx, qweight, scales, zeros, bias, y, ldy, M, N, K, group_size,
                     workspace, workspace_bytes, stream);
}

int w4a16_gemm_f16_noalloc(const w4a16_plan* plan, const void* x, int64_t ldx,
                           const int32_t* qweight, const void* scales, const void* zeros,
                           const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                           int64_t group_size, void* stream) {
  if (int st = check_gemm_shape(M, N, K, group_size)) return st;
  if (int st = check_strides(M, N, K, ldx, ldy)) return st;
  constexpr size_t kMax = W4A16_NOALLOC_SCRATCH_BYTES;
  w4a16_plan p;
  if (plan) {
    // an explicit plan whose partials do not fit the scratch is refused
    p = *plan;
    if (p.flags & ~W4A16_PLAN_ANY_ZEROS) return W4A16_ERR_BAD_PLAN;
    if (plan_scratch_bytes(p, M, N, K) > kMax) return W4A16_ERR_WORKSPACE;
  } else {
    if (int st = auto_plan(x, ldx, qweight, scales, zeros, bias, y, ldy, M, N, K, group_size, &p))
      return st;
    // the automatic plan takes the most k-splits whose partials fit (a plan
    // with one split needs no scratch at all)
    const int32_t flags = p.flags;
    for (int s = p.split_k - 1; plan_scratch_bytes(p, M, N, K) > kMax && s >= 1; --s)
      if (int st = make_plan(M, N, K, group_size, p.kernel, s, &p)) return st;
    p.flags = flags;
    if (plan_scratch_bytes(p, M, N, K) > kMax) return W4A16_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  if (int st = scratch_on_device(&ws)) return st;
  return run_planned(&p, x, ldx, qweight, scales, zeros, bias, y, ldy, M, N, K, group_size, ws,
                     kMax, stream);
}

static int quantize_common(const void* W, bool f32, int32_t* qweight, void* scales, void* zeros,
                           int64_t K, int64_t N, int64_t group_size, int32_t* flag, void* stream) {
  if (int st = check_gemm_shape(0, N, K, group_size)) return st;
  if (K == 0 || N == 0) return W4A16_OK;
  if (!W || !qweight || !scales || !zeros || !flag) return W4A16_ERR_NULL_POINTER;
  return to_status(launch_quantize_pack(W, f32, qweight, scales, zeros, (int)K, (int)N,
                                        (int)group_size, flag,
                                        static_cast<hipStream_t>(stream)));
}

int w4a16_quantize_pack_f16(const void* W, int32_t* qweight, void* scales, void* zeros,
                            int64_t K, int64_t N, int64_t group_size, int32_t* flag,
                            void* stream) {
  return quantize_common(W, false, qweight, scales, zeros, K, N, group_size, flag, stream);
}

int w4a16_quantize_pack_f32(const void* W, int32_t* qweight, void* scales, void* zeros,
                            int64_t K, int64_t N, int64_t group_size, int32_t* flag,
                            void* stream) {
  return quantize_common(W, true, qweight, scales, zeros, K, N, group_size, flag, stream);
}

int w4a16_pack_int4(const int32_t* q, int32_t* qweight, int64_t K, int64_t N, int32_t* flag,
                    void* stream) {
  if (int st = check_gemm_shape(0, N, K, 8)) return st;
  if (K == 0 || N == 0) return W4A16_OK;
  if (!q || !qweight || !flag) return W4A16_ERR_NULL_POINTER;
  return to_status(launch_pack(q, qweight, (int)K, (int)N, flag, static_cast<hipStream_t>(stream)));
}

int w4a16_unpack_int4(const int32_t* qweight, int32_t* q, int64_t K, int64_t N, void* stream) {
  if (int st = check_gemm_shape(0, N, K, 8)) return st;
  if (K == 0 || N == 0) return W4A16_OK;
  if (!q || !qweight) return W4A16_ERR_NULL_POINTER;
  return to_status(launch_unpack(qweight, q, (int)K, (int)N, static_cast<hipStream_t>(stream)));
}

int w4a16_dequantize_f16(const int32_t* qweight, const void* scales, const void* zeros, void* w,
                         int64_t K, int64_t N, int64_t group_size, void* stream) {
  if (int st = check_gemm_shape(0, N, K, group_size)) return st;
  if (K == 0 || N == 0) return W4A16_OK;
  if (!qweight || !scales || !zeros || !w) return W4A16_ERR_NULL_POINTER;
  return to_status(launch_dequant(qweight, scales, zeros, w, (int)K, (int)N, (int)group_size,
                                  static_cast<hipStream_t>(stream)));
}

}  // extern "C"
