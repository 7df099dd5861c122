// Host-side interface between the C-ABI layer (capi.cpp) and the kernel
// translation units.  Internal to libw4a16.so; not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a16 {

// One W4A16 GEMM call: Y[M,N] = X[M,K] @ dequant(qweight, scales, zeros) (+ bias).
// k / G without a division in the kernels: (umulhi(k, magic) + k) >> shift
// with shift = ceil(log2 G) and magic = floor(2^32 (2^shift - G) / G) + 1,
// exact for 0 <= k < 2^31 (magic = 1 for a power of two).
struct GroupDiv {
  uint32_t magic;
  int shift;
};
inline GroupDiv group_div(int G) {
  int l = 0;
  while ((1ll << l) < (long long)G) ++l;
  const uint64_t m = ((1ull << 32) * (uint64_t)((1ll << l) - G)) / (uint64_t)G + 1;
  return GroupDiv{(uint32_t)m, l};
}

struct GemmArgs {
  const void* x;        // fp16 [M, K], rows ldx elements apart
  const int32_t* qw;    // int32 [K/8, N]
  const void* sc;       // fp16 [K/G, N]
  const void* zr;       // fp16 [K/G, N]
  const void* bias;     // fp16 [N] or nullptr
  void* y;              // fp16 [M, N], rows ldy elements apart
  int M, N, K, G;
  int ldx, ldy;         // row strides (>= K, >= N); the vector kernels need
                        // ldx % 8 == 0 and ldy % 4 == 0 (16- / 8-byte rows)
  bool any_zeros = false;   // zeros may be any fp16 value: the fused kernels'
                            // AZ forms (w4a16_device.h); else integers with
                            // |z| <= 1024
};

// Bytes from the first element of x to one past its last: (M - 1) ldx + K
// elements (0 for an empty x).
inline uint64_t x_extent_bytes(const GemmArgs& a) {
  return a.M > 0 && a.K > 0 ? ((uint64_t)(a.M - 1) * (uint64_t)a.ldx + (uint64_t)a.K) * 2u : 0;
}

// Decode GEMV, M <= kGemvMaxM.  A workgroup owns `cols` consecutive columns
// (16, 32, 64, 128 or 256) and K/8/split packed rows; `cfg` picks 8 (cfg 1)
// or 16 (cfg 2, M <= 2) waves per workgroup, cfg 4 / 5 the same with the
// activations staged in LDS (M <= 2; larger M always stages them), cfg 6 / 7
// 16 / 8 waves staged with the dot products on the matrix cores (M <= 2,
// 64- or 128-column blocks); cfg 0 and 3 (4 waves) were retired.  With split > 1,
// `ws` holds the fp32 partials of gemv_workspace_bytes().
constexpr int kGemvMaxM = 8;
// 8 waves per workgroup: two waves per SIMD overlap one wave's dequant with the
// other's outstanding loads; the planner takes 16 waves (cfg 2) for M <= 2 on
// narrow blocks and short rows, where they measured faster on MI355X.
constexpr int kGemvDefaultConfig = 1;
bool gemv_cols_valid(int cols);
bool gemv_cfg_valid(int cfg, int M, int cols);
size_t gemv_workspace_bytes(int M, int N, int K, int split);
int gemv_rows_per_split(int K, int split);
hipError_t launch_gemv(const GemmArgs& a, int cols, int cfg, int split, void* ws,
                       hipStream_t st);

// Prefill GEMM on MFMA.  `cfg` picks the tiling (mfma_tile): 1, 2 (one wave
// per SIMD, 32x32x16), 6 (two waves per SIMD, 32x32x16), 7 (two waves per
// SIMD, 16x16x32, gemm_occ2.hip), 11 / 12 / 13 (128- / 32- / 64-row tiles with
// activations and packed weights streamed into LDS, gemm_stream.hip), 14 (the
// 128-row streamed tile with two k-slices of four waves per workgroup).  Other
// numbers are refused (retired tilings).
struct MfmaTile {
  int bm, bn;
};
constexpr int kMfmaConfigs = 15;
MfmaTile mfma_tile(int cfg);
bool mfma_fits(int M, int N, int K, int G);
// Whether tile configuration `cfg` exists and can run this shape (some need
// K % 64, 128 or 256).
bool mfma_cfg_applicable(int cfg, int M, int N, int K, int G);
// Configurations with a split-K form (fp32 partials, occ2_workspace_bytes()).
bool mfma_cfg_splits(int cfg);
// split > 1 (cfg 7, 11-13 only): fp32 partials in `part`, occ2_workspace_bytes().
hipError_t launch_mfma(const GemmArgs& a, int cfg, int split, float* part, hipStream_t st);
// Split-K epilogue shared by the GEMV and the prefill kernels: y[M, N] =
// fp16(sum of the S fp32 partials [S][M][N], in split order) (+ fp16 bias).
// N % 4 == 0.
hipError_t launch_splitk_reduce(const float* part, const void* bias, void* y, int M, int N, int ldy,
                                int S, hipStream_t st);
// Two-waves-per-SIMD 16x16x32 kernel (mfma cfg 7: 128 x 256): needs K % 64 == 0.
bool occ2_gemm_applicable(int M, int N, int K, int G);
// Split-K of cfg 7: the number of non-empty k-splits for a requested count,
// and the fp32 partial buffer they need (0 when not split).
int occ2_splits(int K, int split);
size_t occ2_workspace_bytes(int M, int N, int K, int split);
// The 128 x 256 tiling of cfg 7 with the packed weights streamed into LDS
// four k-steps ahead (mfma cfg 11), or 32 / 64 x 256 tiles of the same kernel
// (cfg 12 / 13): needs K % 256 == 0.
bool stream_gemm_applicable(int M, int N, int K, int G);
// Splits the streamed kernel makes of a split request (whole 4-step blocks per
// split and k-slice; never more than occ2_splits() for the same request).
int stream_splits(int K, int split, int slices = 1);
// rows = 128, 64 or 32 (tile rows of cfg 11 / 14, 13, 12); slices = 2: two
// k-slices of four waves per workgroup (cfg 14, 128 rows).
hipError_t launch_stream_gemm(const GemmArgs& a, int rows, int split, float* part,
                              hipStream_t st, int slices = 1);
hipError_t launch_occ2_gemm(const GemmArgs& a, int split, float* part, hipStream_t st);

// Buffer-addressed kernels need every operand below 2 GiB.
bool operands_fit(int M, int N, int K, int G);

// Skinny-M GEMM on MFMA (v_mfma_f32_16x16x32_f16), 1 <= M <= kSkinnyMaxM,
// one workgroup per column block and row group over the whole of K (4 waves,
// 8 or 16 when that gives each wave one 256-k batch: K <= 2048 / 4096).
// cfg 0: 16-column blocks (one column per lane, 4-byte weight loads, 2-byte
// scale / zero loads); cfg 2: 32-column blocks (N even: two columns per lane,
// 8-byte weight loads, 4-byte scale / zero loads); cfg 3: 64-column blocks
// (N % 4 == 0: four columns per lane, 16-byte weight loads, 8-byte scale /
// zero loads).  `rows` = rows of y per workgroup: M rounded up to 16 (one
// row group), 16 or 8 (M / 16 or M / 8 row groups); at most 32 on 32-column
// blocks and 16 on 64-column blocks (skinny_plan_valid).  cfg 1 (8 waves in
// the loop) was retired.
constexpr int kSkinnyMaxM = 64;
bool skinny_plan_valid(int cfg, int M, int N, int rows);
hipError_t launch_skinny(const GemmArgs& a, int cfg, int rows, hipStream_t st);

// Sequential-k SIMT kernel: any N, any G dividing K, no alignment needs.
hipError_t launch_simt(const GemmArgs& a, hipStream_t st);

// Quantisation / packing kernels.
hipError_t launch_quantize_pack(const void* W, bool w_is_f32, int32_t* qw, void* sc, void* zr,
                                int K, int N, int G, int32_t* flag, hipStream_t st);
hipError_t launch_pack(const int32_t* q, int32_t* qw, int K, int N, int32_t* flag, hipStream_t st);
hipError_t launch_unpack(const int32_t* qw, int32_t* q, int K, int N, hipStream_t st);
hipError_t launch_dequant(const int32_t* qw, const void* sc, const void* zr, void* w, int K,
                          int N, int G, hipStream_t st);
// flag <- 1 if any of the n fp16 zeros is not an integer in [-1024, 1024].
hipError_t launch_zeros_check(const void* zr, int64_t n, int32_t* flag, hipStream_t st);

}  // namespace w4a16
