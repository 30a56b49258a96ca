// Caller side of the memory sublayer: the `memory_layernorm` in front of the memory
// cross-attention (memory_transformer/memory_block.py:549-558, RMSNorm of :18-28 or
// nn.LayerNorm when use_rms_norm is off).
//
// Forward: one wave per row, the row held in registers (d % 8 == 0, d <= 2048: up to four
// 8-element chunks per lane), one pass over x, y written in the output dtype, the row's
// mean (LayerNorm) and 1/sqrt(var + eps) kept for the backward.
//   RMSNorm:   y = x / sqrt(mean(x^2) + eps) * w          (memory_block.py:26-28)
//   LayerNorm: y = (x - mu) / sqrt(var + eps) * w + b
// Backward: with xh = (x - mu) rstd and g = dy w,
//   dx = rstd (g - mean(g) [LayerNorm only] - xh mean(g xh))   (a row kernel, one wave per row),
//   dw = sum_rows dy xh, db = sum_rows dy                       (a column kernel over row splits,
// then a fixed-order sum over the splits: deterministic).  The two kernels read x and dy once
// each; every launch fills the chip (row-per-wave and column-by-split grids).

#include <algorithm>

#include "moc_common.h"

namespace moc {

constexpr int kNormMaxD = 2048;

template <typename TI>
__device__ __forceinline__ void nload8(const TI* p, float* o) {
  if constexpr (sizeof(TI) == 2) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (float)v[e];
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), c = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = a[e];
      o[4 + e] = c[e];
    }
  }
}

template <typename TO>
__device__ __forceinline__ void nstore8(TO* p, const float* v) {
  if constexpr (sizeof(TO) == 2) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (bf16)v[e];
    *reinterpret_cast<bf16x8*>(p) = r;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

template <typename TX, typename TY, int kCh>
__global__ __launch_bounds__(256) void row_norm_fwd_kernel(const TX* __restrict__ x, int64_t R, int d,
                                                           const float* __restrict__ w, const float* __restrict__ b,
                                                           int layer, float eps, TY* __restrict__ y,
                                                           float* __restrict__ mean_out,
                                                           float* __restrict__ rstd_out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= R) return;
  const int nch = d >> 3;
  const TX* xr = x + r * d;
  float v[kCh][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      nload8<TX>(xr + 8 * c, v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[i][e];
  }
  const float mu = layer ? wave_sum(s) / (float)d : 0.f;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    if (lane + 64 * i < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = v[i][e] - mu;
        q += t * t;
      }
    }
  }
  const float rstd = 1.f / sqrtf(wave_sum(q) / (float)d + eps);
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float wv[8], o[8];
      nload8<float>(w + 8 * c, wv);
      if (layer && b) {
        float bv[8];
        nload8<float>(b + 8 * c, bv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (v[i][e] - mu) * rstd * wv[e] + bv[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (v[i][e] - mu) * rstd * wv[e];
      }
      nstore8<TY>(y + r * d + 8 * c, o);
    }
  }
  if (lane == 0) {
    rstd_out[r] = rstd;
    if (mean_out) mean_out[r] = mu;
  }
}

// dx: one wave per row.
template <typename TX, typename TG, typename TD, int kCh>
__global__ __launch_bounds__(256) void row_norm_bwd_kernel(const TX* __restrict__ x, int64_t R, int d,
                                                           const float* __restrict__ w, int layer,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd, const TG* __restrict__ dy,
                                                           TD* __restrict__ dx) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= R) return;
  const int nch = d >> 3;
  const float mu = layer ? mean[r] : 0.f, rs = rstd[r];
  float xh[kCh][8], g[kCh][8];
  float a = 0.f, c0 = 0.f;
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float wv[8];
      nload8<TX>(x + r * d + 8 * c, xh[i]);
      nload8<TG>(dy + r * d + 8 * c, g[i]);
      nload8<float>(w + 8 * c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) g[i][e] *= wv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xh[i][e] = g[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xh[i][e] = (xh[i][e] - mu) * rs;
      a += g[i][e] * xh[i][e];
      c0 += g[i][e];
    }
  }
  a = wave_sum(a) / (float)d;
  c0 = layer ? wave_sum(c0) / (float)d : 0.f;
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = rs * (g[i][e] - c0 - xh[i][e] * a);
      nstore8<TD>(dx + r * d + 8 * c, o);
    }
  }
}

// part[split][0][j] = sum over the split's kNormColRows rows of dy xh, part[split][1][j] of dy.
// A workgroup owns 256 columns (4 adjacent per thread of a 64-thread column group) and one row
// split; its 4 column groups take interleaved rows and are added in a fixed order.
constexpr int kNormColRows = 64;

template <typename TX, typename TG>
__global__ __launch_bounds__(256) void row_norm_col_kernel(const TX* __restrict__ x, int64_t R, int d, int layer,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd,
                                                           const TG* __restrict__ dy, float* __restrict__ part) {
  __shared__ float4 red[4][64][2];
  const int cq = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int j0 = (blockIdx.x * 64 + cq) * 4;
  const int64_t r0 = (int64_t)blockIdx.y * kNormColRows, r1 = min(R, r0 + kNormColRows);
  float sw[4] = {0.f, 0.f, 0.f, 0.f}, sb[4] = {0.f, 0.f, 0.f, 0.f};
  if (j0 < d) {
    constexpr int kU = 4;
    for (int64_t rb = r0 + grp; rb < r1; rb += 4 * kU) {
      float xv[kU][4], gv[kU][4], mu[kU], rs[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t r = rb + 4 * u;
        const bool live = r < r1;
        mu[u] = (live && layer) ? mean[r] : 0.f;
        rs[u] = live ? rstd[r] : 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[u][e] = gv[u][e] = 0.f;
        if (live) {
          if constexpr (sizeof(TX) == 2) {
            const bf16x4 t = *reinterpret_cast<const bf16x4*>(x + r * d + j0);
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[u][e] = (float)t[e];
          } else {
            const f32x4 t = *reinterpret_cast<const f32x4*>(x + r * d + j0);
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[u][e] = t[e];
          }
          if constexpr (sizeof(TG) == 2) {
            const bf16x4 t = *reinterpret_cast<const bf16x4*>(dy + r * d + j0);
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[u][e] = (float)t[e];
          } else {
            const f32x4 t = *reinterpret_cast<const f32x4*>(dy + r * d + j0);
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[u][e] = t[e];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sw[e] += gv[u][e] * ((xv[u][e] - mu[u]) * rs[u]);
          sb[e] += gv[u][e];
        }
      }
    }
  }
  red[grp][cq][0] = make_float4(sw[0], sw[1], sw[2], sw[3]);
  red[grp][cq][1] = make_float4(sb[0], sb[1], sb[2], sb[3]);
  __syncthreads();
  if (grp == 0 && j0 < d) {
    float4 tw = red[0][cq][0], tb = red[0][cq][1];
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      const float4 a = red[q][cq][0], b = red[q][cq][1];
      tw.x += a.x; tw.y += a.y; tw.z += a.z; tw.w += a.w;
      tb.x += b.x; tb.y += b.y; tb.z += b.z; tb.w += b.w;
    }
    float* dst = part + (int64_t)blockIdx.y * 2 * d;
    *reinterpret_cast<float4*>(dst + j0) = tw;
    *reinterpret_cast<float4*>(dst + d + j0) = tb;
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_row_norm_fwd(int norm, int x_dtype, const void* x, int64_t R, int64_t d, const float* weight,
                     const float* bias, float eps, int y_dtype, void* y, float* mean, float* rstd,
                     hipStream_t stream) {
  MOC_REQUIRE(x && weight && y && rstd, MOC_ERR_ARG, "moc_row_norm_fwd: null pointer");
  MOC_REQUIRE(norm == MOC_NORM_RMS || norm == MOC_NORM_LAYERNORM, MOC_ERR_ARG, "moc_row_norm_fwd: norm %d", norm);
  MOC_REQUIRE(norm == MOC_NORM_RMS || mean, MOC_ERR_ARG, "moc_row_norm_fwd: LayerNorm needs the mean output");
  MOC_REQUIRE(R >= 0 && d > 0 && d % 8 == 0 && d <= kNormMaxD, MOC_ERR_UNSUPPORTED,
              "moc_row_norm_fwd: d=%lld (needs a multiple of 8, <= %d)", (long long)d, kNormMaxD);
  MOC_REQUIRE(eps >= 0.f, MOC_ERR_ARG, "moc_row_norm_fwd: eps < 0");
  if (R == 0) return MOC_OK;
  const int layer = norm == MOC_NORM_LAYERNORM;
  const int kch = (int)((d / 8 + 63) / 64);
  dim3 grid((unsigned)((R + 3) / 4));
#define NF(TX, TY, KC)                                                                                              \
  hipLaunchKernelGGL((row_norm_fwd_kernel<TX, TY, KC>), grid, dim3(256), 0, stream, (const TX*)x, R, (int)d, weight, \
                     bias, layer, eps, (TY*)y, mean, rstd)
#define NFK(TX, TY)   \
  if (kch == 1)       \
    NF(TX, TY, 1);    \
  else if (kch == 2)  \
    NF(TX, TY, 2);    \
  else                \
    NF(TX, TY, 4)
  if (x_dtype == MOC_F32 && y_dtype == MOC_F32) NFK(float, float);
  else if (x_dtype == MOC_F32 && y_dtype == MOC_BF16) NFK(float, bf16);
  else if (x_dtype == MOC_BF16 && y_dtype == MOC_BF16) NFK(bf16, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_row_norm_fwd: dtypes x %d y %d", x_dtype, y_dtype);
#undef NFK
#undef NF
  return check_launch("row_norm_fwd_kernel");
}

size_t moc_row_norm_bwd_workspace(int64_t R, int64_t d) {
  const int64_t nsplit = std::max<int64_t>(1, (R + kNormColRows - 1) / kNormColRows);
  return (size_t)(nsplit * 2 * d) * sizeof(float);
}

int moc_row_norm_bwd(int norm, int x_dtype, const void* x, int64_t R, int64_t d, const float* weight,
                     const float* mean, const float* rstd, int dy_dtype, const void* dy, int dx_dtype, void* dx,
                     float* dweight_dbias, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  MOC_REQUIRE(x && weight && rstd && dy && dx && dweight_dbias && workspace, MOC_ERR_ARG,
              "moc_row_norm_bwd: null pointer");
  MOC_REQUIRE(norm == MOC_NORM_RMS || norm == MOC_NORM_LAYERNORM, MOC_ERR_ARG, "moc_row_norm_bwd: norm %d", norm);
  MOC_REQUIRE(norm == MOC_NORM_RMS || mean, MOC_ERR_ARG, "moc_row_norm_bwd: LayerNorm needs the saved mean");
  MOC_REQUIRE(R >= 0 && d > 0 && d % 8 == 0 && d <= kNormMaxD, MOC_ERR_UNSUPPORTED,
              "moc_row_norm_bwd: d=%lld (needs a multiple of 8, <= %d)", (long long)d, kNormMaxD);
  MOC_REQUIRE(R <= (int64_t)65535 * kNormColRows, MOC_ERR_UNSUPPORTED, "moc_row_norm_bwd: R=%lld rows exceeds %lld",
              (long long)R, (long long)65535 * kNormColRows);
  MOC_REQUIRE(workspace_bytes >= moc_row_norm_bwd_workspace(R, d), MOC_ERR_ARG, "moc_row_norm_bwd: workspace too small");
  if (R == 0) return launch_split_reduce((const float*)workspace, 0, 2 * d, 1.f, dweight_dbias, stream);   // zeros
  const int layer = norm == MOC_NORM_LAYERNORM;
  const int kch = (int)((d / 8 + 63) / 64);
  const int64_t nsplit = (R + kNormColRows - 1) / kNormColRows;
  float* part = (float*)workspace;
  dim3 grid((unsigned)((R + 3) / 4));
  dim3 cgrid((unsigned)((d + 255) / 256), (unsigned)nsplit);
#define NB(TX, TG, TD, KC)                                                                                      \
  hipLaunchKernelGGL((row_norm_bwd_kernel<TX, TG, TD, KC>), grid, dim3(256), 0, stream, (const TX*)x, R, (int)d, \
                     weight, layer, mean, rstd, (const TG*)dy, (TD*)dx)
#define NBK(TX, TG, TD)                                                                                      \
  do {                                                                                                       \
    if (kch == 1)                                                                                            \
      NB(TX, TG, TD, 1);                                                                                     \
    else if (kch == 2)                                                                                       \
      NB(TX, TG, TD, 2);                                                                                     \
    else                                                                                                     \
      NB(TX, TG, TD, 4);                                                                                     \
    hipLaunchKernelGGL((row_norm_col_kernel<TX, TG>), cgrid, dim3(256), 0, stream, (const TX*)x, R, (int)d, layer, \
                       mean, rstd, (const TG*)dy, part);                                                     \
  } while (0)
  if (x_dtype == MOC_F32 && dy_dtype == MOC_F32 && dx_dtype == MOC_F32) NBK(float, float, float);
  else if (x_dtype == MOC_F32 && dy_dtype == MOC_BF16 && dx_dtype == MOC_F32) NBK(float, bf16, float);
  else if (x_dtype == MOC_BF16 && dy_dtype == MOC_BF16 && dx_dtype == MOC_BF16) NBK(bf16, bf16, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_row_norm_bwd: dtypes x %d dy %d dx %d", x_dtype, dy_dtype, dx_dtype);
#undef NBK
#undef NB
  int rc = check_launch("row_norm_bwd_kernel / row_norm_col_kernel");
  if (rc) return rc;
  return launch_split_reduce(part, (int)nsplit, 2 * d, 1.f, dweight_dbias, stream);
}

}  // extern "C"
