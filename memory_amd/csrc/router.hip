// Chapter router kernels: pooling, router linear, softmax + shared-prefix mask
// + top-k + renormalisation, the shared-chapter prepend, and their backwards.
//
// Reference semantics (paths relative to the reference repository root):
//  * pooling            memory_transformer/router.py:96-107 (mean) and
//                       :158-195 (rolling mean; expressed here as a per-position
//                       coefficient vector supplied by the host)
//  * softmax/mask/top-k memory_transformer/router.py:114-149 (sequence level),
//                       :293-329 (token level: slice [S:], renorm, topk, +S)
//  * prepend            memory_transformer/model.py:356-391
// The top-k order is "logit descending, equal logits by ascending chapter id":
// the reference's torch.topk leaves the order of equal values unspecified and
// selects by masked, renormalised fp32 probability, which is a monotone
// function of the logit for a fixed row.
#include "moc_common.h"

namespace moc {

// Monotone map float -> uint32 (larger float => larger key).
__device__ __forceinline__ uint32_t fkey(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int NT>
__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) t += red[i];
  return t;
}
template <int NT>
__device__ __forceinline__ float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = -INFINITY;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) t = fmaxf(t, red[i]);
  return t;
}

constexpr int kRouterThreads = 256;
constexpr int kMaxTopK = 1024;

// Softmax statistics of one row: max, sum of exp(z - max), and the masked sum
// of probabilities over c >= S (probabilities formed as exp(z - max) / Z, the
// same operation order as torch.softmax followed by a masked sum).
struct RowStats { float mx, Z, msum; };

__device__ RowStats row_stats(const float* z, int64_t C, int S, float* red) {
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < C; c += kRouterThreads) m = fmaxf(m, z[c]);
  m = block_reduce_max<kRouterThreads>(m, red);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < C; c += kRouterThreads) s += __expf(z[c] - m);
  const float Z = block_reduce_sum<kRouterThreads>(s, red);
  float ms = 0.f;
  if (S > 0)
    for (int64_t c = S + threadIdx.x; c < C; c += kRouterThreads) ms += __expf(z[c] - m) / Z;
  ms = block_reduce_sum<kRouterThreads>(ms, red);
  return RowStats{m, Z, ms};
}

// One workgroup per row of logits.
__global__ __launch_bounds__(kRouterThreads) void router_topk_kernel(
    const float* __restrict__ logits, int64_t C, int S, int k,
    int32_t* __restrict__ idx_out, float* __restrict__ w_out, float* __restrict__ probs_out) {
  __shared__ float red[kRouterThreads / 64];
  __shared__ int hist[256];
  __shared__ uint32_t sel_key[kMaxTopK];
  __shared__ int32_t sel_idx[kMaxTopK];
  __shared__ float sel_w[kMaxTopK];
  __shared__ int s_state[4];  // prefix, remaining, n_gt counter, running eq
  __shared__ int wave_cnt[kRouterThreads / 64];

  const int64_t r = blockIdx.x;
  const float* z = logits + r * C;
  const int tid = threadIdx.x;
  const RowStats st = row_stats(z, C, S, red);
  const float denom = fmaxf(st.msum, 1e-12f);

  if (probs_out) {
    for (int64_t c = tid; c < C; c += kRouterThreads) probs_out[r * C + c] = __expf(z[c] - st.mx) / st.Z;
  }

  // ---- radix select: exact k-th largest key among c in [S, C)
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int64_t c = S + tid; c < C; c += kRouterThreads) {
      uint32_t u = fkey(z[c]);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid < 64) {
      // lane owns bins 4*lane .. 4*lane+3; suffix sums over bins above.
      int b0 = hist[4 * tid], b1 = hist[4 * tid + 1], b2 = hist[4 * tid + 2], b3 = hist[4 * tid + 3];
      int mine = b0 + b1 + b2 + b3;
      int incl = mine;  // inclusive suffix over lanes >= tid
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        int t = __shfl_down(incl, o, 64);
        if (tid + o < 64) incl += t;
      }
      int above = incl - mine;  // count in bins of lanes > tid
      // walk own bins high to low
      int cnt[4] = {b0, b1, b2, b3};
      int chosen = -1, chosen_above = 0;
      int acc = above;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        if (chosen < 0 && acc < remaining && acc + cnt[j] >= remaining) { chosen = 4 * tid + j; chosen_above = acc; }
        acc += cnt[j];
      }
      if (chosen >= 0) { s_state[0] = chosen; s_state[1] = remaining - chosen_above; }
    }
    __syncthreads();
    prefix |= ((uint32_t)s_state[0]) << shift;
    mask |= 0xFFu << shift;
    remaining = s_state[1];
    __syncthreads();
  }
  const uint32_t thr = prefix;
  const int n_gt = k - remaining;
  if (tid == 0) { s_state[2] = 0; s_state[3] = 0; }
  __syncthreads();
  // ---- collect keys strictly above the threshold (slot order irrelevant: sorted below)
  for (int64_t c = S + tid; c < C; c += kRouterThreads) {
    uint32_t u = fkey(z[c]);
    if (u > thr) {
      int p = atomicAdd(&s_state[2], 1);
      sel_key[p] = u;
      sel_idx[p] = (int32_t)c;
    }
  }
  // ---- collect the `remaining` lowest-index keys equal to the threshold
  const int w = tid >> 6, lane = tid & 63;
  for (int64_t base = S; base < C; base += kRouterThreads) {
    int64_t c = base + tid;
    bool eq = (c < C) && fkey(z[c]) == thr;
    unsigned long long bal = __ballot(eq);
    int rank_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[w] = __popcll(bal);
    __syncthreads();
    int off = s_state[3];
    for (int i = 0; i < w; ++i) off += wave_cnt[i];
    int pos = off + rank_in_wave;
    if (eq && pos < remaining) {
      sel_key[n_gt + pos] = thr;
      sel_idx[n_gt + pos] = (int32_t)c;
    }
    __syncthreads();
    if (tid == 0) {
      int t = 0;
      for (int i = 0; i < kRouterThreads / 64; ++i) t += wave_cnt[i];
      s_state[3] += t;
    }
    __syncthreads();
    if (s_state[3] >= remaining) break;
  }
  __syncthreads();
  // ---- probabilities of the selected chapters, sum, renormalise
  float part = 0.f;
  for (int i = tid; i < k; i += kRouterThreads) {
    float p = __expf(z[sel_idx[i]] - st.mx) / st.Z;
    if (S > 0) p = p / denom;
    sel_w[i] = p;
    part += p;
  }
  const float W = fmaxf(block_reduce_sum<kRouterThreads>(part, red), 1e-12f);
  // ---- rank sort: (key desc, index asc)
  for (int i = tid; i < k; i += kRouterThreads) {
    const uint32_t ki = sel_key[i];
    const int32_t ii = sel_idx[i];
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      uint32_t kj = sel_key[j];
      rank += (kj > ki) || (kj == ki && sel_idx[j] < ii);
    }
    idx_out[r * k + rank] = ii;
    w_out[r * k + rank] = sel_w[i] / W;
  }
}

// dlogits for the chain  p = softmax(z); q = p masked to c >= S; p' = q / clamp(sum q);
// w = p'[idx]; w_hat = w / clamp(sum w).  dw_hat is the incoming gradient.  Mirrors
// autograd of memory_transformer/router.py:114-149 including the clamp_min(1e-12) gates.
__global__ __launch_bounds__(kRouterThreads) void router_topk_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ idx, const float* __restrict__ dw_hat,
    int64_t C, int S, int k, float* __restrict__ dlogits) {
  __shared__ float red[kRouterThreads / 64];
  __shared__ float s_dwraw[kMaxTopK];
  const int64_t r = blockIdx.x;
  const float* z = logits + r * C;
  float* dz = dlogits + r * C;
  const int tid = threadIdx.x;
  const RowStats st = row_stats(z, C, S, red);
  const float denom = fmaxf(st.msum, 1e-12f);
  const bool denom_live = st.msum >= 1e-12f;

  // w_raw and its sum
  float part = 0.f, gw = 0.f;
  for (int i = tid; i < k; i += kRouterThreads) {
    float p = __expf(z[idx[r * k + i]] - st.mx) / st.Z;
    if (S > 0) p = p / denom;
    part += p;
    gw += dw_hat[r * k + i] * p;
  }
  const float Wsum = block_reduce_sum<kRouterThreads>(part, red);
  const float GW = block_reduce_sum<kRouterThreads>(gw, red);  // sum_j g_j w_raw_j
  const float W = fmaxf(Wsum, 1e-12f);
  const bool W_live = Wsum >= 1e-12f;
  // dw_raw_i = g_i / W - [live] * GW / W^2 ; A = sum_i dw_raw_i * q_{idx_i}
  float a = 0.f;
  for (int i = tid; i < k; i += kRouterThreads) {
    float dwr = dw_hat[r * k + i] / W - (W_live ? GW / (W * W) : 0.f);
    s_dwraw[i] = dwr;
    float p = __expf(z[idx[r * k + i]] - st.mx) / st.Z;
    a += dwr * p;
  }
  const float A = block_reduce_sum<kRouterThreads>(a, red);
  __syncthreads();
  // dp_c: dense.  First pass writes dp into dz and accumulates sum_c dp_c p_c.
  float dpp = 0.f;
  for (int64_t c = tid; c < C; c += kRouterThreads) {
    float dp = 0.f;
    if (S > 0) {
      if (c >= S) dp = -(denom_live ? A / (denom * denom) : 0.f);
    }
    dz[c] = dp;
  }
  __syncthreads();
  for (int i = tid; i < k; i += kRouterThreads) {
    int c = idx[r * k + i];
    dz[c] += (S > 0) ? s_dwraw[i] / denom : s_dwraw[i];
  }
  __threadfence_block();
  __syncthreads();
  for (int64_t c = tid; c < C; c += kRouterThreads) dpp += dz[c] * (__expf(z[c] - st.mx) / st.Z);
  const float DPP = block_reduce_sum<kRouterThreads>(dpp, red);
  for (int64_t c = tid; c < C; c += kRouterThreads) {
    float p = __expf(z[c] - st.mx) / st.Z;
    dz[c] = p * (dz[c] - DPP);
  }
}

// omega = [1..1 (S), scale * w] / clamp(sum); idx_star = [0..S-1, idx].
__global__ void prepend_kernel(const int32_t* __restrict__ idx, const float* __restrict__ w, int64_t R,
                               int k, int S, float scale, int32_t* __restrict__ idx_star,
                               float* __restrict__ omega) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (r >= R) return;
  const int lane = threadIdx.x;  // 64 lanes per row
  const int NS = S + k;
  float s = 0.f;
  for (int j = lane; j < NS; j += 64) s += (j < S) ? 1.f : scale * w[r * k + (j - S)];
  s = fmaxf(wave_sum(s), 1e-12f);
  for (int j = lane; j < NS; j += 64) {
    float a = (j < S) ? 1.f : scale * w[r * k + (j - S)];
    omega[r * NS + j] = a / s;
    idx_star[r * NS + j] = (j < S) ? j : idx[r * k + (j - S)];
  }
}

__global__ void prepend_bwd_kernel(const float* __restrict__ w, const float* __restrict__ domega, int64_t R,
                                   int k, int S, float scale, float* __restrict__ dw) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (r >= R) return;
  const int lane = threadIdx.x;
  const int NS = S + k;
  float s = 0.f, g = 0.f;
  for (int j = lane; j < NS; j += 64) {
    float a = (j < S) ? 1.f : scale * w[r * k + (j - S)];
    s += a;
    g += domega[r * NS + j] * a;
  }
  s = wave_sum(s);
  g = wave_sum(g);
  const float D = fmaxf(s, 1e-12f);
  const float corr = (s >= 1e-12f) ? g / (D * D) : 0.f;
  for (int j = S + lane; j < NS; j += 64) dw[r * k + (j - S)] = scale * (domega[r * NS + j] / D - corr);
}

// pooled[b, :] = sum_l coef[l] * h[b, l, :]   (coef == nullptr: mean over L).
// grid (ceil(d/256), B, nsplit); partials [nsplit][B][d] reduced by pool_reduce.
template <typename T>
__global__ __launch_bounds__(256) void pool_partial_kernel(const T* __restrict__ h, int64_t L, int64_t d,
                                                           const float* __restrict__ coef, int rows_per_split,
                                                           float* __restrict__ part) {
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = blockIdx.y;
  const int split = blockIdx.z;
  if (col >= d) return;
  const int64_t l0 = (int64_t)split * rows_per_split;
  const int64_t l1 = min((int64_t)L, l0 + rows_per_split);
  const T* hb = h + b * L * d + col;
  float acc = 0.f;
  if (coef) {
    for (int64_t l = l0; l < l1; ++l) acc += coef[l] * to_f(hb[l * d]);
  } else {
    for (int64_t l = l0; l < l1; ++l) acc += to_f(hb[l * d]);
  }
  part[((int64_t)split * gridDim.y + b) * d + col] = acc;
}

__global__ void pool_reduce_kernel(const float* __restrict__ part, int nsplit, int64_t B, int64_t d, float inv,
                                   float* __restrict__ pooled) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * d) return;
  float s = 0.f;
  for (int j = 0; j < nsplit; ++j) s += part[(int64_t)j * B * d + i];
  pooled[i] = s * inv;
}

// logits[r, c] = x[r, :] . W[c, :] + b[c]; one wave per chapter row, all R rows.
template <typename TW>
__global__ __launch_bounds__(256) void router_linear_kernel(const float* __restrict__ x, int64_t R, int64_t d,
                                                            const TW* __restrict__ W, const float* __restrict__ bias,
                                                            int64_t C, float* __restrict__ logits) {
  const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= C) return;
  const TW* wr = W + c * d;
  const float bc = bias ? bias[c] : 0.f;
  for (int64_t r = 0; r < R; ++r) {
    const float* xr = x + r * d;
    float acc = 0.f;
    for (int64_t j = lane; j < d; j += 64) acc += xr[j] * to_f(wr[j]);
    acc = wave_sum(acc);
    if (lane == 0) logits[r * C + c] = acc + bc;
  }
}

// Backward of the router linear for small R.
//   dW[c, :] = sum_r dz[r, c] x[r, :]     db[c] = sum_r dz[r, c]
//   dx partials over chapter splits, reduced by pool_reduce_kernel.
__global__ __launch_bounds__(256) void router_linear_dw_kernel(const float* __restrict__ dz, const float* __restrict__ x,
                                                               int64_t R, int64_t d, int64_t C,
                                                               float* __restrict__ dW, float* __restrict__ db) {
  const int64_t c = blockIdx.x;
  for (int64_t j = threadIdx.x; j < d; j += 256) {
    float acc = 0.f;
    for (int64_t r = 0; r < R; ++r) acc += dz[r * C + c] * x[r * d + j];
    dW[c * d + j] = acc;
  }
  if (threadIdx.x == 0 && db) {
    float s = 0.f;
    for (int64_t r = 0; r < R; ++r) s += dz[r * C + c];
    db[c] = s;
  }
}

// dx partials: each thread owns one column j and up to kDxRows rows; W is read
// once per row-chunk.  grid (ceil(d/256), nsplit over C, ceil(R/kDxRows)).
constexpr int kDxRows = 16;
template <typename TW>
__global__ __launch_bounds__(256) void router_linear_dx_partial_kernel(const float* __restrict__ dz, const TW* __restrict__ W,
                                                                       int64_t R, int64_t d, int64_t C, int c_per_split,
                                                                       float* __restrict__ part) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int split = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.z * kDxRows;
  const int nr = (int)min((int64_t)kDxRows, R - r0);
  if (j >= d) return;
  const int64_t c0 = (int64_t)split * c_per_split;
  const int64_t c1 = min(C, c0 + c_per_split);
  float acc[kDxRows];
#pragma unroll
  for (int r = 0; r < kDxRows; ++r) acc[r] = 0.f;
  for (int64_t c = c0; c < c1; ++c) {
    const float wv = to_f(W[c * d + j]);
#pragma unroll
    for (int r = 0; r < kDxRows; ++r)
      if (r < nr) acc[r] += dz[(r0 + r) * C + c] * wv;
  }
#pragma unroll
  for (int r = 0; r < kDxRows; ++r)
    if (r < nr) part[((int64_t)split * R + r0 + r) * d + j] = acc[r];
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_router_topk(const float* logits, int64_t R, int64_t C, int S, int k, int32_t* idx, float* w,
                    float* probs, hipStream_t stream) {
  MOC_REQUIRE(logits && idx && w, MOC_ERR_ARG, "moc_router_topk: null pointer");
  MOC_REQUIRE(R >= 0 && C > 0, MOC_ERR_ARG, "moc_router_topk: bad shape R=%lld C=%lld", (long long)R, (long long)C);
  MOC_REQUIRE(S >= 0 && S <= C, MOC_ERR_ARG, "exclude_prefix_chapters must be in [0, %lld], got %d", (long long)C, S);
  MOC_REQUIRE(k > 0 && k <= C - S, MOC_ERR_ARG, "moc_router_topk: k=%d must be in [1, C-S=%lld]", k, (long long)(C - S));
  MOC_REQUIRE(k <= kMaxTopK, MOC_ERR_UNSUPPORTED, "moc_router_topk: k=%d exceeds %d", k, kMaxTopK);
  if (R == 0) return MOC_OK;
  hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)R), dim3(kRouterThreads), 0, stream, logits, C, S, k, idx, w, probs);
  return check_launch("router_topk_kernel");
}

int moc_router_topk_bwd(const float* logits, const int32_t* idx, const float* dw, int64_t R, int64_t C, int S, int k,
                        float* dlogits, hipStream_t stream) {
  MOC_REQUIRE(logits && idx && dw && dlogits, MOC_ERR_ARG, "moc_router_topk_bwd: null pointer");
  MOC_REQUIRE(S >= 0 && S <= C && k > 0 && k <= C - S && k <= kMaxTopK, MOC_ERR_ARG,
              "moc_router_topk_bwd: bad S=%d k=%d C=%lld", S, k, (long long)C);
  if (R == 0) return MOC_OK;
  hipLaunchKernelGGL(router_topk_bwd_kernel, dim3((unsigned)R), dim3(kRouterThreads), 0, stream, logits, idx, dw, C, S, k, dlogits);
  return check_launch("router_topk_bwd_kernel");
}

int moc_prepend_shared(const int32_t* idx, const float* w, int64_t R, int k, int S, float scale, int32_t* idx_star,
                       float* omega, hipStream_t stream) {
  MOC_REQUIRE(idx_star && omega && (k == 0 || (idx && w)), MOC_ERR_ARG, "moc_prepend_shared: null pointer");
  MOC_REQUIRE(S > 0 && k >= 0, MOC_ERR_ARG, "moc_prepend_shared: needs S > 0 (S=%d) and k >= 0", S);
  if (R == 0) return MOC_OK;
  dim3 blk(64, 4);
  hipLaunchKernelGGL(prepend_kernel, dim3((unsigned)((R + 3) / 4)), blk, 0, stream, idx, w, R, k, S, scale, idx_star, omega);
  return check_launch("prepend_kernel");
}

int moc_prepend_shared_bwd(const float* w, const float* domega, int64_t R, int k, int S, float scale, float* dw,
                           hipStream_t stream) {
  MOC_REQUIRE(w && domega && dw, MOC_ERR_ARG, "moc_prepend_shared_bwd: null pointer");
  MOC_REQUIRE(S > 0 && k > 0, MOC_ERR_ARG, "moc_prepend_shared_bwd: needs S > 0 and k > 0");
  if (R == 0) return MOC_OK;
  dim3 blk(64, 4);
  hipLaunchKernelGGL(prepend_bwd_kernel, dim3((unsigned)((R + 3) / 4)), blk, 0, stream, w, domega, R, k, S, scale, dw);
  return check_launch("prepend_bwd_kernel");
}

size_t moc_router_pool_workspace(int64_t B, int64_t L, int64_t d) {
  int nsplit = (int)((L + 63) / 64);
  if (nsplit > 64) nsplit = 64;
  return (size_t)nsplit * B * d * sizeof(float);
}

int moc_router_pool(const void* h, int dtype, int64_t B, int64_t L, int64_t d, const float* coef, float* pooled,
                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  MOC_REQUIRE(h && pooled && workspace, MOC_ERR_ARG, "moc_router_pool: null pointer");
  MOC_REQUIRE(B >= 0 && L > 0 && d > 0, MOC_ERR_ARG, "moc_router_pool: bad shape");
  MOC_REQUIRE(workspace_bytes >= moc_router_pool_workspace(B, L, d), MOC_ERR_ARG, "moc_router_pool: workspace too small");
  if (B == 0) return MOC_OK;
  int nsplit = (int)((L + 63) / 64);
  if (nsplit > 64) nsplit = 64;
  int rows = (int)((L + nsplit - 1) / nsplit);
  dim3 grid((unsigned)((d + 255) / 256), (unsigned)B, (unsigned)nsplit);
  float* part = (float*)workspace;
  if (dtype == MOC_F32)
    hipLaunchKernelGGL(pool_partial_kernel<float>, grid, dim3(256), 0, stream, (const float*)h, L, d, coef, rows, part);
  else if (dtype == MOC_BF16)
    hipLaunchKernelGGL(pool_partial_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)h, L, d, coef, rows, part);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_pool: dtype %d", dtype);
  int rc = check_launch("pool_partial_kernel");
  if (rc) return rc;
  const float inv = coef ? 1.f : 1.f / (float)L;
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((B * d + 255) / 256)), dim3(256), 0, stream, part, nsplit, B, d, inv, pooled);
  return check_launch("pool_reduce_kernel");
}

int moc_router_linear(const float* x, int64_t R, int64_t d, const void* W, int w_dtype, const float* bias, int64_t C,
                      float* logits, hipStream_t stream) {
  MOC_REQUIRE(x && W && logits, MOC_ERR_ARG, "moc_router_linear: null pointer");
  MOC_REQUIRE(R >= 0 && d > 0 && C > 0, MOC_ERR_ARG, "moc_router_linear: bad shape");
  if (R == 0) return MOC_OK;
  dim3 grid((unsigned)((C + 3) / 4));
  if (w_dtype == MOC_F32)
    hipLaunchKernelGGL(router_linear_kernel<float>, grid, dim3(256), 0, stream, x, R, d, (const float*)W, bias, C, logits);
  else if (w_dtype == MOC_BF16)
    hipLaunchKernelGGL(router_linear_kernel<bf16>, grid, dim3(256), 0, stream, x, R, d, (const bf16*)W, bias, C, logits);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_linear: dtype %d", w_dtype);
  return check_launch("router_linear_kernel");
}

size_t moc_router_linear_bwd_workspace(int64_t R, int64_t d, int64_t C) {
  int nsplit = (int)((C + 127) / 128);
  return (size_t)nsplit * R * d * sizeof(float);
}

int moc_router_linear_bwd(const float* dz, const float* x, int64_t R, int64_t d, const void* W, int w_dtype, int64_t C,
                          float* dx, float* dW, float* db, void* workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  MOC_REQUIRE(dz && x && W, MOC_ERR_ARG, "moc_router_linear_bwd: null pointer");
  if (R == 0) return MOC_OK;
  if (dW) {
    hipLaunchKernelGGL(router_linear_dw_kernel, dim3((unsigned)C), dim3(256), 0, stream, dz, x, R, d, C, dW, db);
    int rc = check_launch("router_linear_dw_kernel");
    if (rc) return rc;
  }
  if (dx) {
    MOC_REQUIRE(workspace && workspace_bytes >= moc_router_linear_bwd_workspace(R, d, C), MOC_ERR_ARG,
                "moc_router_linear_bwd: workspace too small");
    int nsplit = (int)((C + 127) / 128);
    dim3 grid((unsigned)((d + 255) / 256), (unsigned)nsplit, (unsigned)((R + kDxRows - 1) / kDxRows));
    float* part = (float*)workspace;
    if (w_dtype == MOC_F32)
      hipLaunchKernelGGL(router_linear_dx_partial_kernel<float>, grid, dim3(256), 0, stream, dz, (const float*)W, R, d, C, 128, part);
    else if (w_dtype == MOC_BF16)
      hipLaunchKernelGGL(router_linear_dx_partial_kernel<bf16>, grid, dim3(256), 0, stream, dz, (const bf16*)W, R, d, C, 128, part);
    else
      return set_error(MOC_ERR_UNSUPPORTED, "moc_router_linear_bwd: dtype %d", w_dtype);
    int rc = check_launch("router_linear_dx_partial_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((R * d + 255) / 256)), dim3(256), 0, stream, part, nsplit, R, d, 1.f, dx);
    return check_launch("pool_reduce_kernel");
  }
  return MOC_OK;
}

}  // extern "C"
