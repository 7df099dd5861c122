// Host-side AddressSanitizer driver for the C ABI of libw4a16 (test
// infrastructure: built and run by tests/test_abi_asan.py on the CPU, no GPU).
//
// It links a build of the library whose host code (capi.cpp: argument checks,
// planner, status strings, workspace sizing) is compiled with
// -fsanitize=address, and calls every entry point of include/w4a16.h along
// the paths that return before any device work: null pointers, bad shapes and
// group sizes, missing or short workspaces, plans that do not fit, plus the
// plan / workspace queries over a grid of shapes and every status string.  A
// heap or stack overflow, use after free or similar in those paths stops the
// run with an ASan report; a wrong status code fails it with a message.
#include "w4a16.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

int g_failures = 0;

void expect(bool ok, const char* what, long long a = 0, long long b = 0) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s (%lld, %lld)\n", what, a, b);
    ++g_failures;
  }
}

// Aligned fake device pointers: never dereferenced on the paths below.
void* fake(uintptr_t v) { return reinterpret_cast<void*>(v); }

}  // namespace

int main() {
  expect(w4a16_abi_version() == W4A16_ABI_VERSION, "abi version");
  const char* id = w4a16_build_id();
  expect(id != nullptr && std::strlen(id) == 64, "build id is a sha256 hex string");

  // every status string, and codes past the enum
  for (int c = -10; c <= 10; ++c) {
    const char* s = w4a16_status_string(c);
    expect(s != nullptr && std::strlen(s) > 0, "status string", c);
  }
  expect(w4a16_status_string(1 << 30) != nullptr, "status string, large code");
  expect(w4a16_status_string(-(1 << 30)) != nullptr, "status string, large negative code");

  // plan and workspace queries over a grid of shapes (kernel families forced
  // too), including zero sizes, ragged N and the largest accepted values
  const int64_t Ms[] = {0, 1, 2, 3, 8, 16, 17, 32, 64, 65, 256, 1024, 4096};
  const int64_t Ns[] = {0, 1, 4, 12, 260, 1028, 4096, 14336, 28672, 65536};
  const int64_t KGs[][2] = {{0, 32}, {8, 8}, {64, 32}, {96, 32}, {4096, 128}, {4096, 64},
                            {14336, 128}, {28672, 32}, {2112, 96}};
  long long plans = 0;
  for (int64_t M : Ms)
    for (int64_t N : Ns)
      for (const auto& kg : KGs)
        for (int32_t kernel = 0; kernel <= 4; ++kernel)
          for (int32_t split : {0, 1, 2, 3, 7, 16}) {
            w4a16_plan p;
            std::memset(&p, 0xA5, sizeof p);
            const int st = w4a16_gemm_plan(M, N, kg[0], kg[1], kernel, split, &p);
            ++plans;
            if (st == W4A16_OK) {
              expect(p.kernel >= 1 && p.kernel <= 4, "planned kernel family", p.kernel);
              expect(p.split_k >= 1, "planned split", p.split_k);
              expect(p.workspace_bytes >= 0, "planned workspace", p.workspace_bytes);
            } else {
              expect(st < 0, "plan error is a negative status", st);
            }
          }
  for (int64_t M : Ms)
    for (int64_t N : Ns)
      for (const auto& kg : KGs) (void)w4a16_gemm_workspace_bytes(M, N, kg[0], kg[1]);
  // out-of-range sizes and group sizes
  w4a16_plan p;
  expect(w4a16_gemm_plan(-1, 4, 8, 8, 0, 0, &p) == W4A16_ERR_BAD_SHAPE, "negative M");
  expect(w4a16_gemm_plan(1, 4, 12, 4, 0, 0, &p) == W4A16_ERR_BAD_SHAPE, "K % 8");
  expect(w4a16_gemm_plan(1, 4, (int64_t)1 << 40, 128, 0, 0, &p) == W4A16_ERR_BAD_SHAPE,
         "K > INT32_MAX");
  expect(w4a16_gemm_plan(1, 4, 64, 0, 0, 0, &p) == W4A16_ERR_BAD_GROUP, "G = 0");
  expect(w4a16_gemm_plan(1, 4, 64, 48, 0, 0, &p) == W4A16_ERR_BAD_GROUP, "K % G");
  expect(w4a16_gemm_plan(1, 4, 64, 32, 9, 0, &p) == W4A16_ERR_BAD_PLAN, "unknown kernel");
  expect(w4a16_gemm_plan(1, 4, 64, 32, 0, 0, nullptr) == W4A16_ERR_NULL_POINTER, "null plan");

  // GEMM entry points: refused before any device work
  void* x = fake(1 << 12);
  const int32_t* qw = static_cast<const int32_t*>(fake(2 << 12));
  void* s = fake(3 << 12);
  void* z = fake(4 << 12);
  void* y = fake(5 << 12);
  expect(w4a16_gemm_f16(nullptr, qw, s, z, y, 4, 64, 64, 32, nullptr, 0, nullptr) ==
             W4A16_ERR_NULL_POINTER, "gemm null x");
  expect(w4a16_gemm_f16(x, qw, s, z, nullptr, 4, 64, 64, 32, nullptr, 0, nullptr) ==
             W4A16_ERR_NULL_POINTER, "gemm null y");
  expect(w4a16_gemm_f16(x, qw, s, z, y, 4, 64, 60, 32, nullptr, 0, nullptr) ==
             W4A16_ERR_BAD_SHAPE, "gemm K % 8");
  expect(w4a16_gemm_f16(x, qw, s, z, y, 4, 64, 64, 24, nullptr, 0, nullptr) ==
             W4A16_ERR_BAD_GROUP, "gemm K % G");
  expect(w4a16_gemm_f16(x, qw, s, z, y, 0, 64, 64, 32, nullptr, 0, nullptr) == W4A16_OK,
         "gemm M = 0 launches nothing");
  expect(w4a16_linear_f16(x, qw, s, z, nullptr, nullptr, 4, 64, 64, 32, nullptr, 0, nullptr) ==
             W4A16_ERR_NULL_POINTER, "linear null y");
  // a forced split plan without its workspace, then with too little of it
  w4a16_plan sp;
  expect(w4a16_gemm_plan(1, 1024, 4096, 128, W4A16_KERNEL_GEMV, 4, &sp) == W4A16_OK,
         "forced split plan");
  expect(sp.workspace_bytes > 0, "split plan needs a workspace", sp.workspace_bytes);
  expect(w4a16_gemm_f16_planned(&sp, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128, nullptr, 0,
                                nullptr) == W4A16_ERR_WORKSPACE, "split plan, no workspace");
  expect(w4a16_gemm_f16_planned(&sp, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128, fake(6 << 12),
                                (size_t)sp.workspace_bytes - 1, nullptr) == W4A16_ERR_WORKSPACE,
         "split plan, short workspace");
  expect(w4a16_gemm_f16_planned(&sp, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128,
                                fake((6 << 12) + 8), (size_t)sp.workspace_bytes, nullptr) ==
             W4A16_ERR_WORKSPACE, "split plan, misaligned workspace");
  expect(w4a16_gemm_f16_planned(nullptr, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128, nullptr, 0,
                                nullptr) == W4A16_ERR_NULL_POINTER, "planned null plan");
  // plans that do not fit their shape
  w4a16_plan bad = sp;
  bad.tile_cfg = 99;
  expect(w4a16_gemm_f16_planned(&bad, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128,
                                fake(6 << 12), (size_t)sp.workspace_bytes, nullptr) ==
             W4A16_ERR_BAD_PLAN, "plan with an unknown tile cfg");
  bad = sp;
  bad.split_k = 1 << 20;
  expect(w4a16_gemm_f16_planned(&bad, x, qw, s, z, nullptr, y, 1, 1024, 4096, 128,
                                fake(6 << 12), (size_t)1 << 40, nullptr) < 0,
         "plan with a split beyond K / 8");
  w4a16_plan sk;
  expect(w4a16_gemm_plan(40, 1024, 4096, 128, W4A16_KERNEL_SKINNY, 0, &sk) == W4A16_OK,
         "skinny plan");
  for (int rows : {0, 4, 48, 64}) {
    w4a16_plan b2 = sk;
    b2.tile_cfg = 3;
    b2.tile_m = rows;
    expect(w4a16_gemm_f16_planned(&b2, x, qw, s, z, nullptr, y, 40, 1024, 4096, 128, nullptr, 0,
                                  nullptr) == W4A16_ERR_BAD_PLAN, "skinny rows", rows);
  }
  // row strides
  expect(w4a16_gemm_f16_strided(nullptr, x, 60, qw, s, z, nullptr, y, 64, 4, 64, 64, 32, nullptr,
                                0, nullptr) == W4A16_ERR_BAD_SHAPE, "ldx < K");
  expect(w4a16_gemm_f16_strided(nullptr, x, 64, qw, s, z, nullptr, y, 60, 4, 64, 64, 32, nullptr,
                                0, nullptr) == W4A16_ERR_BAD_SHAPE, "ldy < N");
  expect(w4a16_gemm_f16_strided(nullptr, x, (int64_t)1 << 40, qw, s, z, nullptr, y, 64, 4, 64, 64,
                                32, nullptr, 0, nullptr) == W4A16_ERR_BAD_SHAPE, "ldx too large");
  // the allocation-free entry point: plans whose partials exceed its scratch
  w4a16_plan big;
  expect(w4a16_gemm_plan(4096, 28672, 28672, 128, W4A16_KERNEL_MFMA, 16, &big) == W4A16_OK,
         "large forced split plan");
  expect(w4a16_gemm_f16_noalloc(&big, x, 28672, qw, s, z, nullptr, y, 28672, 4096, 28672, 28672,
                                128, nullptr) == W4A16_ERR_WORKSPACE, "noalloc scratch too small");
  expect(w4a16_gemm_f16_noalloc(nullptr, x, 60, qw, s, z, nullptr, y, 64, 4, 64, 64, 32,
                                nullptr) == W4A16_ERR_BAD_SHAPE, "noalloc ldx < K");

  // quantise / pack / unpack / dequantise: refused before any device work
  int32_t* q32 = static_cast<int32_t*>(fake(7 << 12));
  int32_t* flag = static_cast<int32_t*>(fake(8 << 12));
  expect(w4a16_quantize_pack_f16(nullptr, q32, s, z, 128, 64, 128, flag, nullptr) ==
             W4A16_ERR_NULL_POINTER, "quantize null W");
  expect(w4a16_quantize_pack_f16(x, q32, s, z, 128, 64, 128, nullptr, nullptr) ==
             W4A16_ERR_NULL_POINTER, "quantize null flag");
  expect(w4a16_quantize_pack_f32(x, q32, s, z, 100, 64, 128, flag, nullptr) ==
             W4A16_ERR_BAD_SHAPE, "quantize K % 8");
  expect(w4a16_quantize_pack_f16(x, q32, s, z, 128, 64, 48, flag, nullptr) ==
             W4A16_ERR_BAD_GROUP, "quantize K % G");
  expect(w4a16_quantize_pack_f16(x, q32, s, z, 0, 64, 128, flag, nullptr) == W4A16_OK,
         "quantize K = 0 launches nothing");
  expect(w4a16_pack_int4(nullptr, q32, 64, 64, flag, nullptr) == W4A16_ERR_NULL_POINTER,
         "pack null q");
  expect(w4a16_pack_int4(q32, q32, 60, 64, flag, nullptr) == W4A16_ERR_BAD_SHAPE, "pack K % 8");
  expect(w4a16_unpack_int4(nullptr, q32, 64, 64, nullptr) == W4A16_ERR_NULL_POINTER,
         "unpack null qweight");
  expect(w4a16_unpack_int4(q32, q32, -8, 64, nullptr) == W4A16_ERR_BAD_SHAPE, "unpack K < 0");
  expect(w4a16_dequantize_f16(q32, s, z, nullptr, 64, 64, 32, nullptr) ==
             W4A16_ERR_NULL_POINTER, "dequantize null w");
  expect(w4a16_dequantize_f16(q32, s, z, y, 64, 64, 0, nullptr) == W4A16_ERR_BAD_GROUP,
         "dequantize G = 0");

  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("abi_driver ok: %lld plans queried\n", plans);
  return 0;
}
