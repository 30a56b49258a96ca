// Chapter plan: de-duplicates the chapters selected across a batch and builds
// the inverted index (chapter -> list of routing edges) that the
// chapter-centric kernels walk.
//
// An "edge" is one (row, slot) pair of a selection matrix, encoded as
// e = row * NS + slot.  Given chap[e] in [0, C):
//   uniq[u]        sorted distinct chapter ids, u < n_uniq
//   edge_u[e]      u such that uniq[u] == chap[e]
//   csr_off[u]     first position of chapter uniq[u] in csr_edge (csr_off[n_uniq] =
//                  number of valid edges)
//   n_uniq[0..1]   number of distinct chapters, number of edges with an id
//                  outside [0, C) (those edges get edge_u = -1 and are skipped,
//                  as the reference kernels skip them: kernels-final/kernel_v4.py:353)
//   csr_edge[p]    edges sorted by (chapter, e) -- a stable counting sort, so the
//                  result (and every accumulation that walks it) is deterministic.
// The reference's inverted index for the weighted kernel does the same with an
// argsort on (b*H + h)*M + chapter (kernels-final/kernel_v4.py:213-257).
#include "moc_common.h"

#include <mutex>

namespace moc {

constexpr int kPlanEdgesPerBlock = 1024;
constexpr int kPlanMaxC = 16384;  // histogram lives in LDS (64 KB)

// counts[g][c] for the edge range of block g.
__global__ __launch_bounds__(256) void plan_hist_kernel(const int32_t* __restrict__ chap, int64_t E, int64_t C,
                                                        int32_t* __restrict__ counts) {
  extern __shared__ int32_t h[];
  const int g = blockIdx.x;
  for (int64_t c = threadIdx.x; c < C; c += 256) h[c] = 0;
  __syncthreads();
  const int64_t e0 = (int64_t)g * kPlanEdgesPerBlock;
  const int64_t e1 = min(E, e0 + kPlanEdgesPerBlock);
  for (int64_t e = e0 + threadIdx.x; e < e1; e += 256) {
    int32_t c = chap[e];
    if (c >= 0 && c < C) atomicAdd(&h[c], 1);  // out-of-range ids are dropped (counted below)
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < C; c += 256) counts[(int64_t)g * C + c] = h[c];
}

// Column prefix over blocks: counts[g][c] <- sum_{g' < g} counts[g'][c]; total[c] = sum.  A
// workgroup per 64 columns (lane = column), wave w of kScanWaves owning blocks [w gq, (w + 1) gq):
// its counts are read at once, the waves' sums scanned through LDS, then each wave writes its
// blocks' prefixes.
constexpr int kScanWaves = 16;
constexpr int kScanPer = 16;   // blocks a wave holds in registers per pass

__global__ __launch_bounds__(64 * kScanWaves) void plan_colscan_kernel(int32_t* __restrict__ counts, int G, int64_t C,
                                                                       int32_t* __restrict__ total) {
  __shared__ int32_t wsum[kScanWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int gq = (G + kScanWaves - 1) / kScanWaves;
  const int g0 = wave * gq, g1 = min(G, g0 + gq);
  int32_t s = 0;
  if (c < C)
    for (int g = g0; g < g1; g += kScanPer) {
      int32_t v[kScanPer];
#pragma unroll
      for (int u = 0; u < kScanPer; ++u) v[u] = g + u < g1 ? counts[(int64_t)(g + u) * C + c] : 0;
#pragma unroll
      for (int u = 0; u < kScanPer; ++u) s += v[u];
    }
  wsum[wave][lane] = s;
  __syncthreads();
  int32_t run = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kScanWaves; ++w) {
    const int32_t t = wsum[w][lane];
    run += w < wave ? t : 0;
    all += t;
  }
  if (c >= C) return;
  if (wave == 0) total[c] = all;
  for (int g = g0; g < g1; g += kScanPer) {
    int32_t v[kScanPer];
#pragma unroll
    for (int u = 0; u < kScanPer; ++u) v[u] = g + u < g1 ? counts[(int64_t)(g + u) * C + c] : 0;
#pragma unroll
    for (int u = 0; u < kScanPer; ++u) {
      if (g + u < g1) counts[(int64_t)(g + u) * C + c] = run;
      run += v[u];
    }
  }
}

// Single workgroup: exclusive scans of total[c] and of (total[c] > 0).
//   start[c] = first csr position of chapter c; uid[c] = unique index of c.
__global__ __launch_bounds__(1024) void plan_scan_kernel(const int32_t* __restrict__ total, int64_t C, int64_t E,
                                                         int32_t* __restrict__ start, int32_t* __restrict__ uid,
                                                         int32_t* __restrict__ uniq, int32_t* __restrict__ csr_off,
                                                         int32_t* __restrict__ n_uniq) {
  __shared__ int32_t s_tot[1024], s_cnt[1024];
  __shared__ int32_t carry[2];
  const int tid = threadIdx.x;
  if (tid == 0) { carry[0] = 0; carry[1] = 0; }
  __syncthreads();
  for (int64_t base = 0; base < C; base += 1024) {
    const int64_t c = base + tid;
    const int32_t t = (c < C) ? total[c] : 0;
    const int32_t f = t > 0 ? 1 : 0;
    s_tot[tid] = t;
    s_cnt[tid] = f;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      int32_t a = (tid >= o) ? s_tot[tid - o] : 0;
      int32_t b = (tid >= o) ? s_cnt[tid - o] : 0;
      __syncthreads();
      s_tot[tid] += a;
      s_cnt[tid] += b;
      __syncthreads();
    }
    const int32_t ex_t = carry[0] + s_tot[tid] - t;
    const int32_t ex_f = carry[1] + s_cnt[tid] - f;
    if (c < C) {
      start[c] = ex_t;
      uid[c] = f ? ex_f : -1;
      if (f) { uniq[ex_f] = (int32_t)c; csr_off[ex_f] = ex_t; }
    }
    __syncthreads();
    if (tid == 1023) { carry[0] += s_tot[1023]; carry[1] += s_cnt[1023]; }
    __syncthreads();
  }
  // n_uniq[1] = number of edges whose chapter id was out of range (they are skipped).
  if (tid == 0) { n_uniq[0] = carry[1]; n_uniq[1] = (int32_t)(E - carry[0]); csr_off[carry[1]] = carry[0]; }
}

// Stable placement: an edge's position is its chapter's start, plus the edges of that chapter in
// earlier blocks, plus the edges of that chapter earlier in this block.  The last term from LDS:
// the block's edges are counted per chapter (arrival order, atomics), the counts scanned into
// per-chapter segments of a block-local list filled in arrival order, and an edge's rank is the
// number of its segment's entries with a smaller index (segments hold ~E / (G C) edges).
__device__ __forceinline__ int plan_wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

__global__ __launch_bounds__(256) void plan_place_kernel(const int32_t* __restrict__ chap, int64_t E, int64_t C,
                                                         const int32_t* __restrict__ counts,
                                                         const int32_t* __restrict__ start,
                                                         const int32_t* __restrict__ uid,
                                                         int32_t* __restrict__ edge_u, int32_t* __restrict__ csr_edge) {
  extern __shared__ int32_t boff[];   // [C]: this block's count, then segment offset, per chapter
  __shared__ int32_t ids[kPlanEdgesPerBlock], slot[kPlanEdgesPerBlock], lst[kPlanEdgesPerBlock];
  __shared__ int32_t wtot[4];
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t e0 = (int64_t)g * kPlanEdgesPerBlock;
  const int n = (int)min((int64_t)kPlanEdgesPerBlock, E - e0);
  for (int64_t c = tid; c < C; c += 256) boff[c] = 0;
  for (int i = tid; i < n; i += 256) ids[i] = chap[e0 + i];
  __syncthreads();
  for (int i = tid; i < n; i += 256) {
    const int32_t c = ids[i];
    slot[i] = (c >= 0 && c < C) ? atomicAdd(&boff[c], 1) : -1;
  }
  __syncthreads();
  // exclusive scan of the per-chapter counts: thread t owns chapters [t per, (t + 1) per)
  const int per = (int)((C + 255) / 256);
  const int64_t c0 = (int64_t)tid * per, c1 = min(C, c0 + per);
  int lt = 0;
  for (int64_t c = c0; c < c1; ++c) lt += boff[c];
  const int it = plan_wave_incl_scan(lt);
  if (lane == 63) wtot[wave] = it;
  __syncthreads();
  int run = it - lt;
  for (int w = 0; w < wave; ++w) run += wtot[w];
  for (int64_t c = c0; c < c1; ++c) {
    const int t = boff[c];
    boff[c] = run;
    run += t;
  }
  __syncthreads();
  for (int i = tid; i < n; i += 256)
    if (slot[i] >= 0) lst[boff[ids[i]] + slot[i]] = i;
  __syncthreads();
  const int placed = wtot[0] + wtot[1] + wtot[2] + wtot[3];
  for (int i = tid; i < n; i += 256) {
    const int32_t c = ids[i];
    const bool ok = c >= 0 && c < C;
    edge_u[e0 + i] = ok ? uid[c] : -1;
    if (!ok) continue;
    const int s0 = boff[c], s1 = c + 1 < C ? boff[c + 1] : placed;
    int before = 0;
    for (int j = s0; j < s1; ++j) before += lst[j] < i;
    csr_edge[start[c] + counts[(int64_t)g * C + c] + before] = (int32_t)(e0 + i);
  }
}

// Whole plan in one workgroup for small batches (E <= 1024 edges, C <= 8192): the
// histogram, both scans and the stable placement run out of LDS, so the plan
// costs one launch instead of four (the sequence-level path has B * (S + k)
// edges, 520 at the paper shape).  Same outputs as the general path.
constexpr int kPlanSmallE = 1024;
constexpr int kPlanSmallC = 8192;

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

__global__ __launch_bounds__(1024) void plan_small_kernel(const int32_t* __restrict__ chap, int64_t E, int64_t C,
                                                          int32_t* __restrict__ uniq, int32_t* __restrict__ n_uniq,
                                                          int32_t* __restrict__ edge_u,
                                                          int32_t* __restrict__ csr_off,
                                                          int32_t* __restrict__ csr_edge) {
  extern __shared__ int32_t lds[];
  int32_t* cnt = lds;          // [C] counts, then first csr position of each chapter
  int32_t* uid = lds + C;      // [C] unique index of each present chapter
  int32_t* fill = lds + 2 * C;  // [C] edges placed so far
  __shared__ int32_t ids[kPlanSmallE];
  __shared__ int32_t tmp[kPlanSmallE];
  __shared__ int32_t wsum[2][16];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int64_t c = tid; c < C; c += 1024) {
    cnt[c] = 0;
    fill[c] = 0;
  }
  if (tid < E) ids[tid] = chap[tid];
  __syncthreads();
  if (tid < E) {
    const int32_t c = ids[tid];
    if (c >= 0 && c < C) atomicAdd(&cnt[c], 1);  // out-of-range ids are dropped (counted below)
  }
  __syncthreads();
  // thread t owns bins [t * per, (t + 1) * per): local totals, block exclusive scan
  const int per = (int)((C + 1023) / 1024);
  const int64_t c0 = (int64_t)tid * per, c1 = min(C, c0 + per);
  int lt = 0, lf = 0;
  for (int64_t c = c0; c < c1; ++c) { lt += cnt[c]; lf += cnt[c] > 0; }
  const int it = wave_incl_scan(lt), iff = wave_incl_scan(lf);
  if (lane == 63) { wsum[0][wave] = it; wsum[1][wave] = iff; }
  __syncthreads();
  int ot = 0, of = 0, tot_t = 0, tot_f = 0;
  for (int w = 0; w < 16; ++w) {
    if (w < wave) { ot += wsum[0][w]; of += wsum[1][w]; }
    tot_t += wsum[0][w];
    tot_f += wsum[1][w];
  }
  int rt = ot + it - lt, rf = of + iff - lf;  // exclusive prefix of this thread's bins
  for (int64_t c = c0; c < c1; ++c) {
    const int t = cnt[c];
    if (t > 0) {
      uniq[rf] = (int32_t)c;
      csr_off[rf] = rt;
      uid[c] = rf;
      ++rf;
    }
    cnt[c] = rt;
    rt += t;
  }
  if (tid == 0) { n_uniq[0] = tot_f; n_uniq[1] = (int32_t)(E - tot_t); csr_off[tot_f] = tot_t; }
  __syncthreads();
  // placement into the chapter's segment in arrival order, then the stable order: an edge's
  // slot is the segment start plus the number of the segment's edges with a smaller id
  const int32_t c = tid < E ? ids[tid] : -1;
  const bool ok = c >= 0 && c < C;
  if (ok) tmp[cnt[c] + atomicAdd(&fill[c], 1)] = tid;
  __syncthreads();
  if (tid < E) {
    edge_u[tid] = ok ? uid[c] : -1;
    if (ok) {
      const int s0 = cnt[c], n = fill[c];
      int before = 0;
      for (int j = 0; j < n; ++j) before += tmp[s0 + j] < tid;
      csr_edge[s0 + before] = tid;
    }
  }
}

// Workspace of moc_chapter_plan_noalloc: a fixed device array (each GPU holds its own copy for
// the life of the process).  Host code never passes `scratch` itself to a kernel -- in host
// code the name is a stand-in, not a device address -- but the address hipGetSymbolAddress
// returns for the current device, looked up once per device and kept.
constexpr size_t kPlanScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kPlanScratchBytes];

constexpr int kPlanMaxDevices = 64;
static std::mutex scratch_mu;
static void* scratch_ptr[kPlanMaxDevices];

// This device's address of `scratch` (looked up on the first call on the device).
static int plan_scratch(void** out) {
  int dev = 0;
  MOC_HIP(hipGetDevice(&dev));
  MOC_REQUIRE(dev >= 0 && dev < kPlanMaxDevices, MOC_ERR_UNSUPPORTED, "moc_chapter_plan_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    MOC_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MOC_REQUIRE(p != nullptr, MOC_ERR_LAUNCH, "moc_chapter_plan_noalloc: no device address for the scratch array");
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return MOC_OK;
}

size_t plan_workspace_bytes(int64_t E, int64_t C) {
  const int64_t G = (E + kPlanEdgesPerBlock - 1) / kPlanEdgesPerBlock;
  // counts[G][C] + total[C] + start[C] + uid[C]
  return (size_t)(G * C + 3 * C) * sizeof(int32_t);
}

// The plan's kernels on a given workspace (every word of it is written before it is read).
int plan_launch(const int32_t* chap, int64_t E, int64_t C, void* workspace, int32_t* uniq, int32_t* n_uniq,
                int32_t* edge_u, int32_t* csr_off, int32_t* csr_edge, hipStream_t stream) {
  if (E <= kPlanSmallE && C <= kPlanSmallC) {
    hipLaunchKernelGGL(plan_small_kernel, dim3(1), dim3(1024), 3 * (size_t)C * sizeof(int32_t), stream, chap, E, C,
                       uniq, n_uniq, edge_u, csr_off, csr_edge);
    return check_launch("plan_small_kernel");
  }
  const int G = (int)((E + kPlanEdgesPerBlock - 1) / kPlanEdgesPerBlock);
  int32_t* counts = (int32_t*)workspace;
  int32_t* total = counts + (int64_t)G * C;
  int32_t* start = total + C;
  int32_t* uid = start + C;
  const size_t lds = (size_t)C * sizeof(int32_t);  // histogram of plan_hist_kernel
  hipLaunchKernelGGL(plan_hist_kernel, dim3(G), dim3(256), lds, stream, chap, E, C, counts);
  int rc = check_launch("plan_hist_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(plan_colscan_kernel, dim3((unsigned)((C + 63) / 64)), dim3(64 * kScanWaves), 0, stream, counts, G,
                     C, total);
  if ((rc = check_launch("plan_colscan_kernel"))) return rc;
  hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(1024), 0, stream, total, C, E, start, uid, uniq, csr_off, n_uniq);
  if ((rc = check_launch("plan_scan_kernel"))) return rc;
  hipLaunchKernelGGL(plan_place_kernel, dim3(G), dim3(256), lds, stream, chap, E, C, counts, start, uid, edge_u,
                     csr_edge);
  return check_launch("plan_place_kernel");
}

}  // namespace moc

using namespace moc;

extern "C" {

size_t moc_chapter_plan_workspace(int64_t E, int64_t C) { return plan_workspace_bytes(E, C); }

int moc_chapter_plan(const int32_t* chap, int64_t E, int64_t C, void* workspace, size_t workspace_bytes,
                     int32_t* uniq, int32_t* n_uniq, int32_t* edge_u, int32_t* csr_off, int32_t* csr_edge,
                     hipStream_t stream) {
  MOC_REQUIRE(chap && workspace && uniq && n_uniq && edge_u && csr_off && csr_edge, MOC_ERR_ARG,
              "moc_chapter_plan: null pointer");
  MOC_REQUIRE(E > 0 && E < (int64_t)1 << 31, MOC_ERR_ARG, "moc_chapter_plan: E=%lld out of range", (long long)E);
  MOC_REQUIRE(C > 0 && C <= kPlanMaxC, MOC_ERR_UNSUPPORTED, "moc_chapter_plan: C=%lld not in [1, %d]", (long long)C,
              kPlanMaxC);
  MOC_REQUIRE(workspace_bytes >= moc_chapter_plan_workspace(E, C), MOC_ERR_ARG, "moc_chapter_plan: workspace too small");
  return plan_launch(chap, E, C, workspace, uniq, n_uniq, edge_u, csr_off, csr_edge, stream);
}

int moc_chapter_plan_noalloc(const int32_t* chap, int64_t E, int64_t C, int32_t* uniq, int32_t* n_uniq,
                             int32_t* edge_u, int32_t* csr_off, int32_t* csr_edge, hipStream_t stream) {
  MOC_REQUIRE(chap && uniq && n_uniq && edge_u && csr_off && csr_edge, MOC_ERR_ARG,
              "moc_chapter_plan_noalloc: null pointer");
  MOC_REQUIRE(E > 0 && E < (int64_t)1 << 31, MOC_ERR_ARG, "moc_chapter_plan_noalloc: E=%lld out of range",
              (long long)E);
  MOC_REQUIRE(C > 0 && C <= kPlanMaxC, MOC_ERR_UNSUPPORTED, "moc_chapter_plan_noalloc: C=%lld not in [1, %d]",
              (long long)C, kPlanMaxC);
  const size_t need = plan_workspace_bytes(E, C);
  MOC_REQUIRE(need <= kPlanScratchBytes, MOC_ERR_UNSUPPORTED,
              "moc_chapter_plan_noalloc: E=%lld edges over C=%lld chapters need %zu bytes of workspace, more than "
              "the %zu-byte fixed scratch (use moc_chapter_plan with a caller workspace)",
              (long long)E, (long long)C, need, kPlanScratchBytes);
  void* ws = nullptr;
  if (int rc = plan_scratch(&ws)) return rc;
  return plan_launch(chap, E, C, ws, uniq, n_uniq, edge_u, csr_off, csr_edge, stream);
}

}  // extern "C"
