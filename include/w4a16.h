/*
 * libw4a16 -- C ABI of the MI355X (gfx950) W4A16 fused dequant-GEMM.
 *
 * Plain C types only: device pointers as `void*` / `int32_t*`, sizes as int64_t,
 * the HIP stream as `void*` (a hipStream_t; NULL = the legacy default stream).
 * All device pointers belong to the calling thread's current HIP device and are
 * owned by the caller; the library allocates nothing and keeps no global mutable
 * state apart from a per-device cache of the CU count and, for
 * w4a16_gemm_f16_noalloc only, a static device scratch array per GPU.
 * Launches are asynchronous on `stream`.
 *
 * Return value: 0 (W4A16_OK) on success, a negative w4a16_status for an invalid
 * argument (detected on the host, before anything is launched), or a positive
 * hipError_t from the launch.
 *
 * Tensor formats (reference: w4a16-kernel/src/w4a16/quant.py:1-30,
 * W4A16_SPEC.md:109-171), all row-major and contiguous:
 *   x       fp16  [M, K]        activations (row stride ldx, w4a16_gemm_f16_strided)
 *   qweight int32 [K/8, N]      word (i, n) holds rows 8i..8i+7, row 8i+j in
 *                               bits [4j, 4j+4), unsigned codes 0..15
 *   scales  fp16  [K/G, N]
 *   zeros   fp16  [K/G, N]      zero-points; W = fp16(fp16(fp16(q) - z) * s)
 *   y       fp16  [M, N]        Y = fp16(fp32-accumulated X @ dequant(W)) (row stride ldy)
 *
 * Zero-points: quantize_weight produces integers 0..15.  By default the fused
 * kernels assume integer zeros with |z| <= 1024, which lets them dequantise
 * with one subtract and one multiply per pair of weights.  Any other zeros
 * (fractions, larger magnitudes, NaN, infinities) need a plan with
 * W4A16_PLAN_ANY_ZEROS set, which runs the same kernels with one more packed
 * subtract per pair and gives the reference's rounding for every fp16 zero;
 * w4a16_zeros_check_f16 tells which a tensor needs.  (The Python layer checks
 * each zeros tensor once and sets the flag itself.)
 */
#ifndef W4A16_H_
#define W4A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_ABI_VERSION 2

enum w4a16_status {
  W4A16_OK = 0,
  W4A16_ERR_NULL_POINTER = -1, /* a required pointer is NULL                     */
  W4A16_ERR_BAD_SHAPE = -2,    /* negative size, K % 8 != 0, or size > INT32_MAX  */
  W4A16_ERR_BAD_GROUP = -3,    /* group_size <= 0 or K % group_size != 0          */
  W4A16_ERR_WORKSPACE = -4,    /* workspace NULL or smaller than the plan needs    */
  W4A16_ERR_BAD_PLAN = -5,     /* plan does not fit the shape / pointers           */
  W4A16_ERR_NO_DEVICE = -6     /* no HIP device could be queried                   */
};

/* Kernel families a plan can name. */
enum w4a16_kernel {
  W4A16_KERNEL_AUTO = 0,
  W4A16_KERNEL_GEMV = 1, /* decode, M <= 8: VALU dequant, dot2 or MFMA dot, split-K */
  W4A16_KERNEL_MFMA = 2, /* prefill: MFMA (32x32x16 / 16x16x32), tile_cfg below     */
  W4A16_KERNEL_SIMT = 3, /* sequential-k, one thread per output, any shape           */
  W4A16_KERNEL_SKINNY = 4 /* small batch: v_mfma_f32_16x16x32_f16, weights streamed   */
};

/* w4a16_plan.flags */
#define W4A16_PLAN_ANY_ZEROS 1 /* zeros may be any fp16 value (see above)     */

/* The launch a GEMM call will make.  Filled by w4a16_gemm_plan(). */
typedef struct w4a16_plan {
  int32_t kernel;          /* enum w4a16_kernel (never AUTO once planned)       */
  int32_t split_k;         /* GEMV, MFMA cfg 7/11-14: k-splits (1 = none)       */
  int32_t tile_cfg;        /* MFMA: tiling 1, 2, 6, 7, 11, 12, 13 or 14
                              (tile_m x tile_n; 14: the 128 x 256 streamed
                              tile with two k-slices per workgroup);
                              GEMV: 1 / 2 = 8 / 16 waves per workgroup
                              (16 for M <= 2), 4 / 5 = the same with the
                              activations staged in LDS (M <= 2; larger M
                              always stages them), 6 / 7 = 16 / 8 waves
                              staged with the dot products on the matrix
                              cores (M <= 2, 64- or 128-column blocks);
                              SKINNY:
                              0 / 2 / 3 = 16 / 32 /
                              64-column blocks (32: N even; 64: N % 4 == 0),
                              4 to 16 waves by K.
                              Other numbers name
                              retired forms and are refused
                              (W4A16_ERR_BAD_PLAN)                           */
  int32_t tile_m, tile_n;  /* workgroup tile; GEMV: 0 x columns per workgroup;
                              SKINNY: rows of y per workgroup (M rounded up
                              to 16, or 16 / 8: one 16- / 8-row group per
                              workgroup, at most 32 on 32-column and 16 on
                              64-column blocks) x columns                    */
  int64_t grid_x, grid_y;  /* workgroups launched                              */
  int64_t workspace_bytes; /* device workspace the call needs (0 = none)        */
  int32_t flags;           /* W4A16_PLAN_ANY_ZEROS or 0 (w4a16_gemm_plan sets
                              0; the caller may set it); other bits are
                              refused (W4A16_ERR_BAD_PLAN)                    */
} w4a16_plan;

/* Version of this ABI (W4A16_ABI_VERSION). */
int w4a16_abi_version(void);

/*
 * Identity of the sources the library was built from: the hex sha256 the build
 * computes over them (never NULL).  No reference counterpart (the reference
 * JIT-compiles its extension on first use, pkg/cuda_kernel.py:56-61); a loader
 * compares it with the sources beside it and refuses a stale library.
 */
const char* w4a16_build_id(void);

/* Static English text for a status code (never NULL). */
const char* w4a16_status_string(int status);

/*
 * Choose the kernel for a GEMM shape on the current device.  `kernel` and
 * `split_k` force a family / k-split when non-zero (tests, benchmarks); 0 lets
 * the library choose.  No reference counterpart: the reference's Triton
 * autotuner picks configs at run time (triton_kernel.py:41-62).
 */
int w4a16_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t group_size, int32_t kernel,
                    int32_t split_k, w4a16_plan* plan);

/*
 * Whether `zeros` (count fp16 values on the device) need W4A16_PLAN_ANY_ZEROS:
 * sets *flag (a device int32 the caller zero-fills) to 1 if any zero is not
 * an integer in [-1024, 1024].  Asynchronous on `stream`.  No reference
 * counterpart: the reference's kernels dequantise every zero alike
 * (triton_kernel.py:117-119, cuda/w4a16_gemm.cu:51-58); here a caller checks a
 * zeros tensor once, when it is made or loaded, not on every GEMM.
 */
int w4a16_zeros_check_f16(const void* zeros, int64_t count, int32_t* flag, void* stream);

/* Workspace bytes the automatic plan for this shape needs (0 = none). */
size_t w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size);

/*
 * Fused W4A16 GEMM, y = x @ dequant(qweight, scales, zeros).
 * Replaces the reference's fused entry point w4a16_matmul
 * (w4a16-kernel/src/w4a16/triton_kernel.py:131-200) and its native launcher
 * w4a16_gemm_cuda (w4a16-kernel/src/w4a16/cuda/w4a16_gemm.cu:76-115).
 * `workspace` (256-byte aligned) must hold w4a16_gemm_workspace_bytes() bytes
 * of fp32 split-K partials; its contents need no initialisation and are
 * overwritten by every call.  Integer zeros with |z| <= 1024 only (any other
 * zeros: a plan with W4A16_PLAN_ANY_ZEROS, w4a16_gemm_f16_strided).  Calls
 * that share one workspace must be ordered (same stream).  M = 0 or N = 0 launches nothing;
 * K = 0 writes y = 0 (x, qweight, scales and zeros may then be NULL).  The
 * library issues kernel launches only (no memset or copy), so calls can be
 * captured into a HIP graph.
 */
int w4a16_gemm_f16(const void* x, const int32_t* qweight, const void* scales, const void* zeros,
                   void* y, int64_t M, int64_t N, int64_t K, int64_t group_size,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * W4A16Linear.forward's arithmetic (w4a16-kernel/src/w4a16/linear.py:82-92):
 * y = fp16(x @ dequant(W)) + bias, the bias added in fp16 after the GEMM's own
 * rounding, fused into the GEMM epilogue.  `bias` may be NULL.
 */
int w4a16_linear_f16(const void* x, const int32_t* qweight, const void* scales,
                     const void* zeros, const void* bias, void* y, int64_t M, int64_t N,
                     int64_t K, int64_t group_size, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Run a GEMM (with optional bias) with an explicit plan from w4a16_gemm_plan(). */
int w4a16_gemm_f16_planned(const w4a16_plan* plan, const void* x, const int32_t* qweight,
                           const void* scales, const void* zeros, const void* bias, void* y,
                           int64_t M, int64_t N, int64_t K, int64_t group_size, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * As w4a16_gemm_f16_planned with row strides: row m of x starts ldx elements
 * after row m-1 (ldx >= K), row m of y ldy elements after row m-1 (ldy >= N),
 * so x and y may be column slices of wider row-major buffers (a fused QKV
 * output, a packed activation buffer).  The reference's kernel takes strides
 * (w4a16-kernel/src/w4a16/triton_kernel.py:71-75, 94, 127) but its wrapper
 * asserts contiguity (triton_kernel.py:170-173); this entry point exposes the
 * row-strided case.  `plan` NULL chooses automatically; the vector kernels
 * need ldx % 8 == 0 (and ldy % 4 == 0 where they store 4-column quads: MFMA
 * plans and split-K), else the automatic plan takes the SIMT kernel and an
 * explicit plan is refused (W4A16_ERR_BAD_PLAN).  ldx < K or ldy < N is
 * W4A16_ERR_BAD_SHAPE.  The workspace is that of the same shape unstrided.
 */
int w4a16_gemm_f16_strided(const w4a16_plan* plan, const void* x, int64_t ldx,
                           const int32_t* qweight, const void* scales, const void* zeros,
                           const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                           int64_t group_size, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * Bytes of the device scratch behind w4a16_gemm_f16_noalloc: a static array
 * that every GPU the library runs on holds until the process ends.
 */
#define W4A16_NOALLOC_SCRATCH_BYTES (16u << 20)

/*
 * As w4a16_gemm_f16_strided, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): no workspace argument and no allocation of any kind.  No
 * counterpart in the reference.  The split-K partials go to the library's own
 * static device scratch of W4A16_NOALLOC_SCRATCH_BYTES per GPU (its address is
 * resolved with hipGetSymbolAddress on a device's first call).  An explicit
 * `plan` whose partials exceed that size is refused with W4A16_ERR_WORKSPACE;
 * with `plan` NULL the automatic plan is limited to the most k-splits whose
 * partials fit (one split needs none, so every shape runs).  Every call on a
 * GPU shares that GPU's scratch, which keeps the last call's contents
 * (nothing needs to start zeroed: a call writes its partials before it reads
 * them), so calls that overlap on one GPU -- different streams, or graphs
 * replayed concurrently -- race and must be ordered by the caller.  Results
 * equal w4a16_gemm_f16_strided's for the same plan.  The scratch address a
 * device's first call resolves is kept for the life of the process: do not
 * call this entry point on a device after hipDeviceReset.
 */
int w4a16_gemm_f16_noalloc(const w4a16_plan* plan, const void* x, int64_t ldx,
                           const int32_t* qweight, const void* scales, const void* zeros,
                           const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                           int64_t group_size, void* stream);

/*
 * Group-wise asymmetric uint4 quantisation of fp16 W [K, N] with int4 packing,
 * bit-exact with the reference's quantize_weight evaluated by torch on the CPU
 * (w4a16-kernel/src/w4a16/quant.py:101-144).  `flag` is a device int32 the
 * caller zero-fills; the kernel sets it to 1 if W holds a non-finite value (the
 * reference's pack_int4 range assertion fires for such input, quant.py:62-63).
 */
int w4a16_quantize_pack_f16(const void* W, int32_t* qweight, void* scales, void* zeros,
                            int64_t K, int64_t N, int64_t group_size, int32_t* flag,
                            void* stream);

/*
 * As w4a16_quantize_pack_f16 for fp32 W [K, N]: the reference quantises fp32
 * weights in fp32 without rounding them to fp16 first (quant.py:105,124).
 */
int w4a16_quantize_pack_f32(const void* W, int32_t* qweight, void* scales, void* zeros,
                            int64_t K, int64_t N, int64_t group_size, int32_t* flag,
                            void* stream);

/*
 * pack_int4 (w4a16-kernel/src/w4a16/quant.py:45-70): int32 codes [K, N] ->
 * int32 [K/8, N].  `flag` (caller zero-filled) is set to 1 if a code lies
 * outside [0, 15] (the reference asserts, quant.py:62-63).
 */
int w4a16_pack_int4(const int32_t* q, int32_t* qweight, int64_t K, int64_t N, int32_t* flag,
                    void* stream);

/* unpack_int4 (w4a16-kernel/src/w4a16/quant.py:73-95): int32 [K/8, N] -> int32 [K, N]. */
int w4a16_unpack_int4(const int32_t* qweight, int32_t* q, int64_t K, int64_t N, void* stream);

/*
 * dequantize_weight (w4a16-kernel/src/w4a16/quant.py:147-178):
 * w = fp16((fp16(q) - z) * s), fp16 [K, N]; exact fp16 arithmetic for any zeros.
 */
int w4a16_dequantize_f16(const int32_t* qweight, const void* scales, const void* zeros, void* w,
                         int64_t K, int64_t N, int64_t group_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H_ */
