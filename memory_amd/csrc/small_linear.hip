// y = x W^T for few rows (decode: one token per sequence through q_proj / o_proj,
// memory_attention.py:140-143, :241, :456): x [M][K], W [N][K] bf16, M <= 256.
//
// A library GEMM tiles such a product into a handful of output tiles, each walking the whole
// K dimension on its own, so the launch is one long chain of dependent loads.  Here a
// workgroup owns one 16 x 16 output tile (64 rows x 768 columns make 192 workgroups), and its
// 4 waves split K: each wave issues all of its x and W fragment loads before its first MFMA
// (v_mfma_f32_16x16x32_bf16), and the four partial tiles are added through LDS in a fixed
// order.  Bound: the latency of one round of loads (each W slice is re-read by the M / 16 row
// tiles, mostly from L2).

#include "moc_common.h"

namespace moc {

constexpr int kSlWaves = 4;
constexpr int kSlTiles = 1;       // 16-row MFMA tiles per workgroup
constexpr int kSlRows = 16 * kSlTiles;
constexpr int kSlChunks = 6;      // 32-wide K chunks a wave holds in registers at once

template <typename TO>
__global__ __launch_bounds__(64 * kSlWaves) void small_linear_kernel(const bf16* __restrict__ x, int M, int K,
                                                                    const bf16* __restrict__ W, int N,
                                                                    TO* __restrict__ y) {
  __shared__ f32x4 red[kSlWaves][kSlTiles][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * kSlRows;
  const int kw = K / kSlWaves;                 // this wave's K range: [wave * kw, wave * kw + kw)
  const int nch = kw / 32;
  f32x4 acc[kSlTiles];
#pragma unroll
  for (int mt = 0; mt < kSlTiles; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16* wrow = W + (size_t)(n0 + c16) * K + wave * kw + 8 * g;
  for (int c0 = 0; c0 < nch; c0 += kSlChunks) {
    bf16x8 a[kSlChunks][kSlTiles], b[kSlChunks];
#pragma unroll
    for (int j = 0; j < kSlChunks; ++j) {
      const bool live = c0 + j < nch;
      const int k = 32 * (c0 + j);
      b[j] = live ? *reinterpret_cast<const bf16x8*>(wrow + k) : bf16x8{};
#pragma unroll
      for (int mt = 0; mt < kSlTiles; ++mt) {
        const int m = m0 + 16 * mt + c16;
        a[j][mt] = (live && m < M) ? *reinterpret_cast<const bf16x8*>(x + (size_t)m * K + wave * kw + k + 8 * g)
                                   : bf16x8{};
      }
    }
#pragma unroll
    for (int j = 0; j < kSlChunks; ++j)
#pragma unroll
      for (int mt = 0; mt < kSlTiles; ++mt) mma(acc[mt], a[j][mt], b[j]);
  }
#pragma unroll
  for (int mt = 0; mt < kSlTiles; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();
  // wave t (< kSlTiles) sums tile t of its lane over the waves, in wave order
  const int mt = threadIdx.x >> 6;
  if (mt >= kSlTiles) return;
  f32x4 s = red[0][mt][lane];
#pragma unroll
  for (int w = 1; w < kSlWaves; ++w) {
    const f32x4 v = red[w][mt][lane];
    s = f32x4{s[0] + v[0], s[1] + v[1], s[2] + v[2], s[3] + v[3]};
  }
  // accumulator layout: column c16, rows 4 g + e of the 16-row tile
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = m0 + 16 * mt + 4 * g + e;
    if (m < M) y[(size_t)m * N + n0 + c16] = from_f<TO>(s[e]);
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_linear_rows(const void* x, int64_t M, int64_t K, const void* W, int64_t N, int out_dtype, void* y,
                    hipStream_t stream) {
  MOC_REQUIRE(x && W && y, MOC_ERR_ARG, "moc_linear_rows: null pointer");
  MOC_REQUIRE(M >= 0 && M <= 256 && K > 0 && N > 0, MOC_ERR_UNSUPPORTED,
              "moc_linear_rows: M=%lld (at most 256 rows), K=%lld, N=%lld", (long long)M, (long long)K, (long long)N);
  MOC_REQUIRE(K % (32 * kSlWaves) == 0 && N % 16 == 0 && K <= 65536 && N <= 65536, MOC_ERR_UNSUPPORTED,
              "moc_linear_rows: K=%lld must be a multiple of %d and N=%lld of 16", (long long)K, 32 * kSlWaves,
              (long long)N);
  MOC_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)W & 15) == 0, MOC_ERR_ARG,
              "moc_linear_rows: x and W must be 16-byte aligned");
  if (M == 0) return MOC_OK;
  dim3 grid((unsigned)(N / 16), (unsigned)((M + kSlRows - 1) / kSlRows));
  if (out_dtype == MOC_BF16)
    hipLaunchKernelGGL(small_linear_kernel<bf16>, grid, dim3(64 * kSlWaves), 0, stream, (const bf16*)x, (int)M, (int)K,
                       (const bf16*)W, (int)N, (bf16*)y);
  else if (out_dtype == MOC_F32)
    hipLaunchKernelGGL(small_linear_kernel<float>, grid, dim3(64 * kSlWaves), 0, stream, (const bf16*)x, (int)M,
                       (int)K, (const bf16*)W, (int)N, (float*)y);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_linear_rows: out dtype %d", out_dtype);
  return check_launch("small_linear_kernel");
}

}  // extern "C"
