// AdamW for the chapter bank, dense or row-sparse with an exact lazy catch-up.
//
// The reference steps the whole bank (memory_bank.py:62, an nn.Parameter of N_m = C * T rows)
// with torch.optim.AdamW every step (training/trainer.py:309-392: param group "memory_bank",
// weight decay on; torch >= 2.0, requirements.txt:14, foreach implementation, amsgrad off).
// Per element and step j (lr_j from the schedule, bias corrections bc1_j = 1 - beta1^j,
// bc2_j = 1 - beta2^j):
//   p <- p * (1 - lr_j wd)
//   m <- lerp(m, g, 1 - beta1)
//   v <- v * beta2 + (1 - beta2) g g
//   p <- p + (-lr_j / bc1_j) * m / (sqrt(v) / sqrt(bc2_j) + eps)
// A row whose gradient is zero still changes (the decays and the moment term), so skipping it
// is not the same optimizer.  Here each chunk of kOptChunk elements of a chapter's T * d block
// carries the step it is current to; a chunk that had no gradient for some steps is brought
// forward by replaying those zero-gradient steps in registers (same formulas, the per-step
// scalars from a device history) the next time it is read or stepped.  Touched rows cost HBM
// traffic every step; untouched rows cost nothing until they are read.

#include <algorithm>

#include "moc_common.h"

namespace moc {

constexpr int kOptThreads = 256;
constexpr int kOptPerThread = 8;
constexpr int kOptChunk = kOptThreads * kOptPerThread;   // elements per work item
constexpr int kOptWgPerCu = 8;

// Step-independent constants: the lerp weight 1 - beta1 (and which of torch's two lerp forms
// it selects), beta2, 1 - beta2, eps.
struct AdamWConst {
  float w1, b2, omb2, eps;
  int small_w1;   // |w1| < 0.5: self + w (end - self); else end - (end - self)(1 - w)
};

// Per-step scalars h = {1 - lr wd, -lr / bc1, sqrt(bc2), unused}.
__device__ __forceinline__ float lerp_t(float self, float end, const AdamWConst& k) {
  return k.small_w1 ? self + k.w1 * (end - self) : end - (end - self) * (1.f - k.w1);
}

__device__ __forceinline__ void adamw_elem(float& p, float& m, float& v, float g, float4 h, const AdamWConst& k) {
  p = p * h.x;
  m = lerp_t(m, g, k);
  v = v * k.b2;
  v = v + k.omb2 * (g * g);
  const float den = sqrtf(v) / h.z + k.eps;
  p = p + h.y * (m / den);
}

// One work item = chunk `ch` of chapter c (elements c*T*d + ch*kOptChunk ...).  The chunk is
// brought from its tag t0 to step tz with zero gradients, then (grad != null) step t runs with
// the gradient.  Chapters come from `list` (n_list[0] of them) or are 0 .. n_all-1.
template <bool kMirror>
__global__ __launch_bounds__(kOptThreads) void bank_adamw_kernel(
    float* __restrict__ p, bf16* __restrict__ mirror, float* __restrict__ m, float* __restrict__ v,
    const float* __restrict__ grad, const float* __restrict__ grad_scale, const int32_t* __restrict__ list,
    const int32_t* __restrict__ n_list, int64_t n_all, int64_t chunk_elems, int nchunk, int32_t* __restrict__ tags,
    float4* __restrict__ hist, int t, float4 h_t, AdamWConst k) {
  __shared__ float4 sh[kOptThreads];
  const int tid = threadIdx.x;
  const int64_t n = list ? (int64_t)n_list[0] : n_all;
  const int64_t items = n * nchunk;
  const bool with_grad = grad != nullptr;
  // step t's scalars, read by later launches' catch-up (this launch reads only steps < t)
  if (with_grad && blockIdx.x == 0 && tid == 0) hist[t] = h_t;
  const int tz = with_grad ? t - 1 : t;
  const float gs = (with_grad && grad_scale) ? grad_scale[0] : 1.f;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int64_t u = it / nchunk;
    const int ch = (int)(it - u * nchunk);
    const int64_t c = list ? (int64_t)list[u] : u;
    const int64_t ti = c * nchunk + ch;
    const int t0 = tags[ti];
    if (t0 >= t) continue;   // already current (uniform over the workgroup)
    const int64_t base = c * chunk_elems + (int64_t)ch * kOptChunk;
    const int ne = (int)min((int64_t)kOptChunk, chunk_elems - (int64_t)ch * kOptChunk);
    float pr[kOptPerThread], mr[kOptPerThread], vr[kOptPerThread], gr[kOptPerThread];
#pragma unroll
    for (int x = 0; x < kOptPerThread; ++x) {
      const int i = tid + kOptThreads * x;
      const bool in = i < ne;
      pr[x] = in ? p[base + i] : 0.f;
      mr[x] = in ? m[base + i] : 0.f;
      vr[x] = in ? v[base + i] : 0.f;
      gr[x] = (in && with_grad) ? grad[base + i] * gs : 0.f;
    }
    // zero-gradient steps t0+1 .. tz, their scalars staged through LDS
    for (int j0 = t0 + 1; j0 <= tz; j0 += kOptThreads) {
      const int nj = min(kOptThreads, tz - j0 + 1);
      __syncthreads();
      if (tid < nj) sh[tid] = hist[j0 + tid];
      __syncthreads();
      for (int jj = 0; jj < nj; ++jj) {
        const float4 h = sh[jj];
#pragma unroll
        for (int x = 0; x < kOptPerThread; ++x) adamw_elem(pr[x], mr[x], vr[x], 0.f, h, k);
      }
    }
    if (with_grad) {
#pragma unroll
      for (int x = 0; x < kOptPerThread; ++x) adamw_elem(pr[x], mr[x], vr[x], gr[x], h_t, k);
    }
#pragma unroll
    for (int x = 0; x < kOptPerThread; ++x) {
      const int i = tid + kOptThreads * x;
      if (i < ne) {
        p[base + i] = pr[x];
        m[base + i] = mr[x];
        v[base + i] = vr[x];
        if constexpr (kMirror) mirror[base + i] = (bf16)pr[x];
      }
    }
    if (tid == 0) tags[ti] = t;
  }
}

// list = the chapters whose tag equals `epoch`, ascending; n_list[0] = their number.  One
// workgroup (prefix sums over 1,024-chapter blocks).
__global__ __launch_bounds__(1024) void bank_touched_kernel(const int32_t* __restrict__ chap_epoch, int64_t C,
                                                           int epoch, int32_t* __restrict__ list,
                                                           int32_t* __restrict__ n_list) {
  __shared__ int wsum[16];
  __shared__ int base_s;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) base_s = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < C; c0 += 1024) {
    const int64_t c = c0 + tid;
    const bool hit = c < C && chap_epoch[c] == epoch;
    const uint64_t bal = __ballot(hit);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[w] = __popcll(bal);
    __syncthreads();
    int off = base_s;
    for (int i = 0; i < w; ++i) off += wsum[i];
    if (hit) list[off + before] = (int32_t)c;
    __syncthreads();
    if (tid == 0) {
      int s = 0;
      for (int i = 0; i < 16; ++i) s += wsum[i];
      base_s += s;
    }
    __syncthreads();
  }
  if (tid == 0) n_list[0] = base_s;
}

// part[it] = sum of g^2 over work item it (chapter list[u] or u, chunk ch), in list order.
__global__ __launch_bounds__(kOptThreads) void bank_sqnorm_part_kernel(const float* __restrict__ grad,
                                                                      const int32_t* __restrict__ list,
                                                                      const int32_t* __restrict__ n_list,
                                                                      int64_t n_all, int64_t chunk_elems, int nchunk,
                                                                      float* __restrict__ part) {
  __shared__ float red[kOptThreads / 64];
  const int tid = threadIdx.x;
  const int64_t n = list ? (int64_t)n_list[0] : n_all;
  const int64_t items = n * nchunk;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int64_t u = it / nchunk;
    const int ch = (int)(it - u * nchunk);
    const int64_t c = list ? (int64_t)list[u] : u;
    const int64_t base = c * chunk_elems + (int64_t)ch * kOptChunk;
    const int ne = (int)min((int64_t)kOptChunk, chunk_elems - (int64_t)ch * kOptChunk);
    float s = 0.f;
#pragma unroll
    for (int x = 0; x < kOptPerThread; ++x) {
      const int i = tid + kOptThreads * x;
      const float g = i < ne ? grad[base + i] : 0.f;
      s += g * g;
    }
    s = wave_sum(s);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) part[it] = red[0] + red[1] + red[2] + red[3];
  }
}

// out[0] = sum of part[0 .. n*nchunk) in a fixed order.
__global__ __launch_bounds__(1024) void bank_sqnorm_final_kernel(const float* __restrict__ part,
                                                                const int32_t* __restrict__ n_list, int64_t n_all,
                                                                int nchunk, float* __restrict__ out) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  const int64_t items = (n_list ? (int64_t)n_list[0] : n_all) * nchunk;
  float s = 0.f;
  for (int64_t i = tid; i < items; i += 1024) s += part[i];
  s = wave_sum(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int i = 0; i < 16; ++i) t += red[i];
    out[0] = t;
  }
}

int opt_grid(int64_t max_items) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>(max_items, (int64_t)cus * kOptWgPerCu));
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_bank_chunk_count(int64_t chunk_elems) { return (int)((chunk_elems + kOptChunk - 1) / kOptChunk); }

int moc_bank_adamw(float* param, void* mirror, int mirror_dtype, float* exp_avg, float* exp_avg_sq, const float* grad,
                   const float* grad_scale, const int32_t* list, const int32_t* n_list, int64_t max_list,
                   int64_t num_chapters, int64_t chunk_elems, int32_t* tags, float* hist, int64_t hist_capacity,
                   int step, float decay, float neg_step_size, float bc2_sqrt, float beta1, float beta2, float eps,
                   hipStream_t stream) {
  MOC_REQUIRE(param && exp_avg && exp_avg_sq && tags && hist, MOC_ERR_ARG, "moc_bank_adamw: null pointer");
  MOC_REQUIRE((list == nullptr) == (n_list == nullptr), MOC_ERR_ARG,
              "moc_bank_adamw: list / n_list must be both set or both null");
  MOC_REQUIRE(num_chapters > 0 && chunk_elems > 0, MOC_ERR_ARG, "moc_bank_adamw: bad shape");
  MOC_REQUIRE(step >= 1 && (int64_t)step < hist_capacity, MOC_ERR_ARG,
              "moc_bank_adamw: step %d outside the history capacity %lld", step, (long long)hist_capacity);
  MOC_REQUIRE(mirror == nullptr || mirror_dtype == MOC_BF16, MOC_ERR_UNSUPPORTED,
              "moc_bank_adamw: the mirror must be bf16");
  MOC_REQUIRE(((uintptr_t)hist & 15) == 0, MOC_ERR_ARG, "moc_bank_adamw: hist must be 16-byte aligned");
  MOC_REQUIRE(list == nullptr || (max_list >= 0 && max_list <= num_chapters), MOC_ERR_ARG,
              "moc_bank_adamw: max_list %lld outside [0, %lld]", (long long)max_list, (long long)num_chapters);
  const int nchunk = moc_bank_chunk_count(chunk_elems);
  const int64_t max_items = (list ? max_list : num_chapters) * nchunk;
  if (max_items == 0) {
    if (!grad) return MOC_OK;
  }
  AdamWConst k;
  k.w1 = 1.f - beta1;
  k.small_w1 = fabsf(k.w1) < 0.5f;
  k.b2 = beta2;
  k.omb2 = 1.f - beta2;
  k.eps = eps;
  const float4 h = make_float4(decay, neg_step_size, bc2_sqrt, 0.f);
  const int grid = opt_grid(std::max<int64_t>(max_items, 1));
  if (mirror)
    hipLaunchKernelGGL((bank_adamw_kernel<true>), dim3(grid), dim3(kOptThreads), 0, stream, param, (bf16*)mirror,
                       exp_avg, exp_avg_sq, grad, grad_scale, list, n_list, num_chapters, chunk_elems, nchunk, tags,
                       (float4*)hist, step, h, k);
  else
    hipLaunchKernelGGL((bank_adamw_kernel<false>), dim3(grid), dim3(kOptThreads), 0, stream, param, (bf16*)nullptr,
                       exp_avg, exp_avg_sq, grad, grad_scale, list, n_list, num_chapters, chunk_elems, nchunk, tags,
                       (float4*)hist, step, h, k);
  return check_launch("bank_adamw_kernel");
}

int moc_bank_touched(const int32_t* chap_epoch, int64_t num_chapters, int epoch, int32_t* list, int32_t* n_list,
                     hipStream_t stream) {
  MOC_REQUIRE(chap_epoch && list && n_list, MOC_ERR_ARG, "moc_bank_touched: null pointer");
  MOC_REQUIRE(num_chapters > 0 && num_chapters < ((int64_t)1 << 31), MOC_ERR_ARG, "moc_bank_touched: bad C");
  hipLaunchKernelGGL(bank_touched_kernel, dim3(1), dim3(1024), 0, stream, chap_epoch, num_chapters, epoch, list,
                     n_list);
  return check_launch("bank_touched_kernel");
}

size_t moc_bank_sqnorm_workspace(int64_t max_list, int64_t chunk_elems) {
  return (size_t)std::max<int64_t>(1, max_list * moc_bank_chunk_count(chunk_elems)) * sizeof(float);
}

int moc_bank_sqnorm(const float* grad, const int32_t* list, const int32_t* n_list, int64_t max_list,
                    int64_t chunk_elems, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream) {
  MOC_REQUIRE(grad && out && workspace, MOC_ERR_ARG, "moc_bank_sqnorm: null pointer");
  MOC_REQUIRE((list == nullptr) == (n_list == nullptr), MOC_ERR_ARG,
              "moc_bank_sqnorm: list / n_list must be both set or both null");
  MOC_REQUIRE(max_list >= 0 && chunk_elems > 0, MOC_ERR_ARG, "moc_bank_sqnorm: bad shape");
  MOC_REQUIRE(workspace_bytes >= moc_bank_sqnorm_workspace(max_list, chunk_elems), MOC_ERR_ARG,
              "moc_bank_sqnorm: workspace too small");
  const int nchunk = moc_bank_chunk_count(chunk_elems);
  const int64_t max_items = max_list * nchunk;
  if (max_items > 0) {
    hipLaunchKernelGGL(bank_sqnorm_part_kernel, dim3(opt_grid(max_items)), dim3(kOptThreads), 0, stream, grad, list,
                       n_list, max_list, chunk_elems, nchunk, (float*)workspace);
    const int rc = check_launch("bank_sqnorm_part_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(bank_sqnorm_final_kernel, dim3(1), dim3(1024), 0, stream, (const float*)workspace, n_list,
                     max_list, nchunk, out);
  return check_launch("bank_sqnorm_final_kernel");
}

}  // extern "C"
