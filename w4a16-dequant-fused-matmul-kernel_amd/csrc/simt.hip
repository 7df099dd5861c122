// Sequential-k SIMT W4A16 GEMM: one thread per output element.
//
// MI355X counterpart of the reference's native CUDA kernel
// (w4a16-kernel/src/w4a16/cuda/w4a16_gemm.cu:20-74): per-element fp16 dequant
// (fp16(q) - z) * s and an fp32 fused multiply-add over k in increasing order,
// one rounding to fp16 at the end.  It accepts any N, any G dividing K and
// unaligned pointers, so it also serves shapes the vector kernels do not take.
// It is not a performance path.
#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

__global__ __launch_bounds__(256) void simt_kernel(const f16* __restrict__ X,
                                                   const uint32_t* __restrict__ QW,
                                                   const f16* __restrict__ SC,
                                                   const f16* __restrict__ ZR,
                                                   const f16* __restrict__ bias,
                                                   f16* __restrict__ Y, int M, int N, int K,
                                                   int G, int ldx, int ldy) {
  const int n = blockIdx.x * 64 + (threadIdx.x & 63);
  const int m = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (n >= N || m >= M) return;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const uint32_t w = QW[(size_t)(k >> 3) * N + n];
    const uint32_t q = (w >> (4 * (k & 7))) & 0xFu;
    const int g = k / G;
    const f16 s = SC[(size_t)g * N + n];
    const f16 z = ZR[(size_t)g * N + n];
    const f16 wd = ((f16)(float)q - z) * s;
    acc = __builtin_fmaf((float)X[(size_t)m * ldx + k], (float)wd, acc);
  }
  f16 y = f32_to_f16(acc);
  if (bias) y = y + bias[n];
  Y[(size_t)m * ldy + n] = y;
}

}  // namespace

hipError_t launch_simt(const GemmArgs& a, hipStream_t st) {
  dim3 grid((a.N + 63) / 64, (a.M + 3) / 4);
  hipLaunchKernelGGL(simt_kernel, grid, dim3(256), 0, st, static_cast<const f16*>(a.x),
                     reinterpret_cast<const uint32_t*>(a.qw), static_cast<const f16*>(a.sc),
                     static_cast<const f16*>(a.zr), static_cast<const f16*>(a.bias),
                     static_cast<f16*>(a.y), a.M, a.N, a.K, a.G, a.ldx, a.ldy);
  return hipGetLastError();
}

}  // namespace w4a16
