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

constexpr int kMaxTopK = 1024;
constexpr int kMaxSeqShared = 1024;  // shared chapters of the fused sequence-router backward
constexpr int kMaxRouterC = 16384;  // the row lives in LDS (64 KB)

// Workgroup size per row: rows are few for sequence-level routing (one per
// sequence: latency-bound, so many threads per row) and many for token-level.
inline int router_threads(int64_t R) { return R <= 64 ? 1024 : 256; }

// Loads row z [C] into LDS with every load of a thread in flight before the stores.
template <int NT>
__device__ __forceinline__ void load_row(const float* __restrict__ z, int64_t C, float* zs) {
  int64_t c = threadIdx.x;
  for (; c + 3 * NT < C; c += 4 * NT) {
    const float a = z[c], b = z[c + NT], e = z[c + 2 * NT], f = z[c + 3 * NT];
    zs[c] = a;
    zs[c + NT] = b;
    zs[c + 2 * NT] = e;
    zs[c + 3 * NT] = f;
  }
  for (; c < C; c += NT) zs[c] = z[c];
  __syncthreads();
}

// Softmax statistics of one row (from LDS): max, sum of exp(z - max), and the
// masked sum of probabilities over c >= S (probabilities formed as
// exp(z - max) / Z, the same operation order as torch.softmax followed by a
// masked sum).
struct RowStats { float mx, Z, msum; };

template <int NT>
__device__ RowStats row_stats(const float* zs, int64_t C, int S, float* red) {
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < C; c += NT) m = fmaxf(m, zs[c]);
  m = block_reduce_max<NT>(m, red);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < C; c += NT) s += __expf(zs[c] - m);
  const float Z = block_reduce_sum<NT>(s, red);
  float ms = 0.f;
  if (S > 0) {
    for (int64_t c = S + threadIdx.x; c < C; c += NT) ms += __expf(zs[c] - m) / Z;
    ms = block_reduce_sum<NT>(ms, red);
  }
  return RowStats{m, Z, ms};
}

// omega = [1..1 (S), scale * w] / clamp(sum); idx_star = [0..S-1, idx] for one row, by one
// wave (lane = threadIdx.x % 64): the sum is formed lane-strided and wave-reduced, the order
// prepend_kernel and prepend_row_bwd use.
__device__ __forceinline__ void prepend_row(const int32_t* idx, const float* w, int k, int S, float scale,
                                            int32_t* idx_star, float* omega, int lane) {
  const int NS = S + k;
  float s = 0.f;
  for (int j = lane; j < NS; j += 64) s += (j < S) ? 1.f : scale * w[j - S];
  s = fmaxf(wave_sum(s), 1e-12f);
  for (int j = lane; j < NS; j += 64) {
    const float a = (j < S) ? 1.f : scale * w[j - S];
    omega[j] = a / s;
    idx_star[j] = (j < S) ? j : idx[j - S];
  }
}

// Gradient of prepend_row w.r.t. w for one row (one wave): dw[i] = scale (domega[S+i] / D - corr).
__device__ __forceinline__ void prepend_row_bwd(const float* w, const float* domega, int k, int S, float scale,
                                                float* dw, int lane) {
  const int NS = S + k;
  float s = 0.f, g = 0.f;
  for (int j = lane; j < NS; j += 64) {
    const float a = (j < S) ? 1.f : scale * w[j - S];
    s += a;
    g += domega[j] * a;
  }
  s = wave_sum(s);
  g = wave_sum(g);
  const float D = fmaxf(s, 1e-12f);
  const float corr = (s >= 1e-12f) ? g / (D * D) : 0.f;
  for (int j = S + lane; j < NS; j += 64) dw[j - S] = scale * (domega[j] / D - corr);
}

// Exact k-th largest key among c in [S, C) by an 8-bit radix select over the order-preserving
// keys, then the keys above it and the lowest-id ties at it, into sel_key / sel_idx (any order).
// The top-k kernel's path for rows whose boundary value bin holds too many logits.
template <int NT>
__device__ void radix_select(const float* zs, int64_t C, int S, int k, uint32_t* sel_key, int32_t* sel_idx,
                             int* s_state, int* wave_cnt) {
  __shared__ int hist[256];
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int64_t c = S + tid; c < C; c += NT) {
      const uint32_t u = fkey(zs[c]);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid < 64) {
      // lane owns bins 4*lane .. 4*lane+3; suffix sums over bins above.
      const int b0 = hist[4 * tid], b1 = hist[4 * tid + 1], b2 = hist[4 * tid + 2], b3 = hist[4 * tid + 3];
      const int mine = b0 + b1 + b2 + b3;
      int incl = mine;  // inclusive suffix over lanes >= tid
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_down(incl, o, 64);
        if (tid + o < 64) incl += t;
      }
      const int cnt[4] = {b0, b1, b2, b3};
      int chosen = -1, chosen_above = 0;
      int acc = incl - mine;  // count in bins of lanes > tid
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        if (chosen < 0 && acc < remaining && acc + cnt[j] >= remaining) { chosen = 4 * tid + j; chosen_above = acc; }
        acc += cnt[j];
      }
      if (chosen >= 0) { s_state[0] = chosen; s_state[1] = remaining - chosen_above; s_state[4] = cnt[chosen & 3]; }
    }
    __syncthreads();
    prefix |= ((uint32_t)s_state[0]) << shift;
    mask |= 0xFFu << shift;
    remaining = s_state[1];
    __syncthreads();
  }
  const uint32_t thr = prefix;
  const int n_gt = k - remaining;
  // after the last pass every key of the chosen bin equals thr
  const bool all_ties = s_state[4] == remaining;
  __syncthreads();
  if (tid == 0) { s_state[2] = 0; s_state[3] = 0; }
  __syncthreads();
  // ---- collect keys above the threshold (and every tie when all of them are taken);
  // slot order is irrelevant: the rank sort below fixes it
  for (int64_t c = S + tid; c < C; c += NT) {
    const uint32_t u = fkey(zs[c]);
    if (u > thr || (all_ties && u == thr)) {
      const int p = atomicAdd(&s_state[2], 1);
      sel_key[p] = u;
      sel_idx[p] = (int32_t)c;
    }
  }
  if (!all_ties) {
    // ---- more ties than slots: the `remaining` lowest-index keys equal to the threshold
    const int w = tid >> 6, lane = tid & 63;
    for (int64_t base = S; base < C; base += NT) {
      const int64_t c = base + tid;
      const bool eq = (c < C) && fkey(zs[c]) == thr;
      const unsigned long long bal = __ballot(eq);
      const int rank_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
      if (lane == 0) wave_cnt[w] = __popcll(bal);
      __syncthreads();
      int off = s_state[3];
      for (int i = 0; i < w; ++i) off += wave_cnt[i];
      const int pos = off + rank_in_wave;
      if (eq && pos < remaining) {
        sel_key[n_gt + pos] = thr;
        sel_idx[n_gt + pos] = (int32_t)c;
      }
      __syncthreads();
      if (tid == 0) {
        int t = 0;
        for (int i = 0; i < NT / 64; ++i) t += wave_cnt[i];
        s_state[3] += t;
      }
      __syncthreads();
      if (s_state[3] >= remaining) break;
    }
  }
}

// Ranks of n keys (key descending, chapter id ascending): G lanes of one wave (G a power of two,
// as many as NT threads allow up to 64) share one element's count over j, then emit(i, rank,
// key, id) runs on the group's first lane.
template <int NT, typename Emit>
__device__ __forceinline__ void rank_keys(const uint32_t* key, const int32_t* id, int n, Emit emit) {
  int G = 64;
  while (G > 1 && G * n > NT) G >>= 1;
  const int tid = threadIdx.x, part = tid & (G - 1);
  for (int i0 = 0; i0 < n; i0 += NT / G) {
    const int i = i0 + tid / G;  // the same for the G lanes of a group
    int rank = 0;
    uint32_t ki = 0;
    int32_t ii = 0;
    if (i < n) {
      ki = key[i];
      ii = id[i];
      for (int j = part; j < n; j += G) {
        const uint32_t kj = key[j];
        rank += (kj > ki) || (kj == ki && id[j] < ii);
      }
    }
    for (int o = 1; o < G; o <<= 1) rank += __shfl_xor(rank, o, 64);
    if (i < n && part == 0) emit(i, rank, ki, ii);
  }
}

// Selection by value bins: the selectable logits (c >= S) span [lo, hi]; bin(z) =
// min(kTopkBins - 1, (z - lo) * kTopkBins / (hi - lo)) is non-decreasing in z, so every logit
// in a bin above the bin holding the k-th largest is selected and only that boundary bin's
// logits (a handful for any spread of values) are ranked exactly.
constexpr int kTopkBins = 2048;
constexpr int kTopkCand = 512;  // boundary-bin logits ranked directly; more go to the radix path

__device__ __forceinline__ int topk_bin(float z, float lo, float inv) {
  return min(kTopkBins - 1, (int)((z - lo) * inv));
}

// One workgroup per row of logits; the row is read from HBM once into LDS.
// With idx_star / omega (non-null, S > 0) the kernel also writes the shared-chapter prepend of
// its row (prepend_kernel's values, summed in the same order), so the sequence router's chain
// top-k -> prepend is one launch.
template <int NT>
__global__ __launch_bounds__(NT) void router_topk_kernel(
    const float* __restrict__ logits, int64_t C, int S, int k,
    int32_t* __restrict__ idx_out, float* __restrict__ w_out, float* __restrict__ probs_out,
    float scale, int32_t* __restrict__ idx_star, float* __restrict__ omega) {
  static_assert(kTopkBins % NT == 0, "bins per thread");
  constexpr int BPT = kTopkBins / NT;
  constexpr int NW = NT / 64;
  extern __shared__ float zs[];  // the row, C floats
  __shared__ float red[3][NW];
  __shared__ int hist[kTopkBins];
  __shared__ int wsum[NW];
  __shared__ uint32_t sel_key[kMaxTopK];
  __shared__ int32_t sel_idx[kMaxTopK];
  __shared__ float sorted_w[kMaxTopK];
  __shared__ int32_t sorted_i[kMaxTopK];
  __shared__ uint32_t cand_key[kTopkCand];
  __shared__ int32_t cand_idx[kTopkCand];
  // boundary bin, remaining, logits in it, selected appended, candidates appended, running eq,
  // ties at threshold (radix path)
  __shared__ int s_state[8];
  __shared__ int wave_cnt[NW];

  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  load_row<NT>(logits + r * C, C, zs);

  // ---- max of the row (softmax) and the selectable range [lo, hi]; the histogram is cleared
  // before the reduction's barriers
#pragma unroll
  for (int i = 0; i < BPT; ++i) hist[tid * BPT + i] = 0;
  if (tid < 8) s_state[tid] = 0;
  float mxa = -INFINITY, hi = -INFINITY, lo = INFINITY;
  for (int64_t c = tid; c < C; c += NT) {
    const float z = zs[c];
    mxa = fmaxf(mxa, z);
    if (c >= S) {
      hi = fmaxf(hi, z);
      lo = fminf(lo, z);
    }
  }
  mxa = wave_max(mxa);
  hi = wave_max(hi);
  lo = -wave_max(-lo);
  if (lane == 0) {
    red[0][wv] = mxa;
    red[1][wv] = hi;
    red[2][wv] = lo;
  }
  __syncthreads();
  mxa = red[0][0], hi = red[1][0], lo = red[2][0];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    mxa = fmaxf(mxa, red[0][i]);
    hi = fmaxf(hi, red[1][i]);
    lo = fminf(lo, red[2][i]);
  }
  const float inv = (float)kTopkBins / (hi - lo);
  const bool binned = hi > lo && inv > 0.f && inv < INFINITY;
  __syncthreads();  // red is reused below

  // ---- softmax sums (all chapters; the selectable ones) and the histogram of the selectable
  float s_all = 0.f, s_sel = 0.f;
  for (int64_t c = tid; c < C; c += NT) {
    const float z = zs[c];
    const float e = __expf(z - mxa);
    s_all += e;
    if (c >= S) {
      s_sel += e;
      if (binned) atomicAdd(&hist[topk_bin(z, lo, inv)], 1);
    }
  }
  s_all = wave_sum(s_all);
  s_sel = wave_sum(s_sel);
  if (lane == 0) {
    red[0][wv] = s_all;
    red[1][wv] = s_sel;
  }
  __syncthreads();
  float Z = 0.f, Zs = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    Z += red[0][i];
    Zs += red[1][i];
  }
  // masked probability mass over c >= S (router.py:126-129 renormalisation)
  const RowStats st{mxa, Z, S > 0 ? Zs / Z : 1.f};
  const float denom = fmaxf(st.msum, 1e-12f);

  if (probs_out) {
    for (int64_t c = tid; c < C; c += NT) probs_out[r * C + c] = __expf(zs[c] - st.mx) / st.Z;
  }

  bool exact = false;  // sel_key / sel_idx hold the k selected (any order)
  if (!binned && hi == lo) {
    // every selectable logit is equal: the k lowest chapter ids
    for (int i = tid; i < k; i += NT) {
      sel_key[i] = fkey(hi);
      sel_idx[i] = S + i;
    }
    exact = true;
  } else if (binned) {
    // boundary bin: suffix sums over bins from the top; thread tid owns bins tid*BPT .. +BPT-1
    int cnt[BPT];
    int mine = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      cnt[i] = hist[tid * BPT + i];
      mine += cnt[i];
    }
    // inclusive suffix sum over the wave's lanes >= lane, then over the waves above
    int incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_down(incl, o, 64);
      if (lane + o < 64) incl += t;
    }
    if (lane == 0) wsum[wv] = incl;
    __syncthreads();
    int above = incl - mine;  // bins of higher threads
    for (int i = wv + 1; i < NW; ++i) above += wsum[i];
#pragma unroll
    for (int i = BPT - 1; i >= 0; --i) {
      if (above < k && above + cnt[i] >= k) {
        s_state[0] = tid * BPT + i;
        s_state[1] = k - above;
        s_state[2] = cnt[i];
      }
      above += cnt[i];
    }
    __syncthreads();
    const int bstar = s_state[0], remaining = s_state[1], nb = s_state[2];
    const int n_above = k - remaining;
    if (nb <= kTopkCand) {
      // collect: bins above the boundary are selected, the boundary bin's logits are candidates
      for (int64_t c = S + tid; c < C; c += NT) {
        const float z = zs[c];
        const int b = topk_bin(z, lo, inv);
        if (b > bstar) {
          const int p = atomicAdd(&s_state[3], 1);
          sel_key[p] = fkey(z);
          sel_idx[p] = (int32_t)c;
        } else if (b == bstar) {
          const int p = atomicAdd(&s_state[4], 1);
          cand_key[p] = fkey(z);
          cand_idx[p] = (int32_t)c;
        }
      }
      __syncthreads();
      // the `remaining` best candidates (key descending, chapter id ascending)
      rank_keys<NT>(cand_key, cand_idx, nb, [&](int, int rank, uint32_t ki, int32_t ii) {
        if (rank < remaining) {
          sel_key[n_above + rank] = ki;
          sel_idx[n_above + rank] = ii;
        }
      });
      exact = true;
    }
  }
  if (!exact) {
    radix_select<NT>(zs, C, S, k, sel_key, sel_idx, s_state, wave_cnt);
  }
  __syncthreads();
  // ---- rank sort (key desc, index asc) of the selected chapters with their probabilities;
  // the slots above were filled in atomic order, so everything after this works in rank order
  // (the sum below is then formed the same way on every run)
  rank_keys<NT>(sel_key, sel_idx, k, [&](int, int rank, uint32_t, int32_t ii) {
    float p = __expf(zs[ii] - st.mx) / st.Z;
    if (S > 0) p = p / denom;
    sorted_w[rank] = p;
    sorted_i[rank] = ii;
  });
  __syncthreads();
  // ---- renormalise
  float part = 0.f;
  for (int i = tid; i < k; i += NT) part += sorted_w[i];
  const float W = fmaxf(block_reduce_sum<NT>(part, red[2]), 1e-12f);
  for (int i = tid; i < k; i += NT) {
    const float v = sorted_w[i] / W;
    idx_out[r * k + i] = sorted_i[i];
    w_out[r * k + i] = v;
    sorted_w[i] = v;
  }
  if (!idx_star) return;
  __syncthreads();
  if (tid < 64) prepend_row(sorted_i, sorted_w, k, S, scale, idx_star + r * (S + k), omega + r * (S + k), tid);
}

// --------------------------------------------------- many rows: one wave per row
// Rows of at most 64 * kWaveMaxE logits with k <= 64 (the token-level router: R = B * L rows):
// the row lives in the wave's registers (lane l holds c = l + 64 j), every reduction is across
// lanes, and nothing waits on a workgroup barrier; a workgroup carries kWaveRows independent rows.
constexpr int kWaveMaxE = 72;  // C <= 4,608
// the kernels take E = ceil(C / 64) rounded up to one of these register-row lengths: rows of up
// to 4,160 logits (4,097 chapters) in 65 registers per lane keep the top-k kernel at 157 VGPRs,
// three waves per SIMD instead of two at 72
constexpr int kWaveShortE = 65;
constexpr int kWaveRows = 4;
constexpr int kWaveBins = 1024;
constexpr int kWaveCand = 128;
constexpr int kWaveMaxK = 64;

struct WaveTopkLds {
  int hist[kWaveBins];
  uint32_t sel_key[kWaveMaxK];
  int32_t sel_idx[kWaveMaxK];
  uint32_t cand_key[kWaveCand];
  int32_t cand_idx[kWaveCand];
  float sorted_w[kWaveMaxK];
  int32_t sorted_i[kWaveMaxK];
  int count[2];
};

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ float fkey_inv(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}
// inclusive sum over lanes >= lane
__device__ __forceinline__ int wave_suffix_sum(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_down(v, o, 64);
    if (lane + o < 64) v += t;
  }
  return v;
}

// the lane id through an empty asm: the per-element predicates derived from it are then formed
// inside each loop instead of once for the whole kernel (72 lane masks would stay live in SGPRs)
__device__ __forceinline__ int wave_opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// z[j] = row[lane + 64 j] for j < kWaveMaxE (-inf past C): buffer loads from a per-row resource,
// one lane offset and constant column offsets (no 64-bit address per load)
template <int E>
__device__ __forceinline__ void wave_load_row(const float* row, int C, int lane, float (&z)[E]) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), (short)0, C * 4, 0x00020000);
  const int ln = wave_opaque(lane);   // keeps the 72 column predicates out of loops around the call
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, 256 * j, 0));
    z[j] = ln + 64 * j < C ? v : -INFINITY;
  }
}

// Forward: the selection of router_topk_kernel (value bins over the selectable range, the
// boundary bin's logits ranked exactly; key descending, chapter id ascending) within one wave.
// A boundary bin with more than kWaveCand logits (plateaus of equal or near-equal values) is
// resolved by repeated wave-wide maxima of (key, -id) over its logits, one selection each.
template <int E>
__global__ __launch_bounds__(64 * kWaveRows) void router_topk_wave_kernel(
    const float* __restrict__ logits, int64_t R, int64_t C, int S, int k, int32_t* __restrict__ idx_out,
    float* __restrict__ w_out, float* __restrict__ probs_out, float scale, int32_t* __restrict__ idx_star,
    float* __restrict__ omega) {
  __shared__ WaveTopkLds lds_all[kWaveRows];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r = (int64_t)blockIdx.x * kWaveRows + wv;  // wave-uniform: the row's buffer resources stay scalar
  if (r >= R) return;
  WaveTopkLds& sm = lds_all[wv];
  const int Ci = (int)C;
  float z[E];
  wave_load_row(logits + r * C, Ci, lane, z);
#pragma unroll
  for (int i = 0; i < kWaveBins / 64; ++i) sm.hist[lane * (kWaveBins / 64) + i] = 0;
  if (lane < 2) sm.count[lane] = 0;
  // padding holds -inf: it takes part in no maximum and adds exp(-inf) = 0 to the sums
  float mxa = -INFINITY, hi = -INFINITY, lo = INFINITY;
  int ln = wave_opaque(lane);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int c = ln + 64 * j;
    const bool sel = c < Ci && c >= S;
    mxa = fmaxf(mxa, z[j]);
    hi = fmaxf(hi, sel ? z[j] : -INFINITY);
    lo = fminf(lo, sel ? z[j] : INFINITY);
  }
  const float lane_hi = hi;
  mxa = wave_max(mxa);
  hi = wave_max(hi);
  lo = -wave_max(-lo);
  float s_all = 0.f, s_sel = 0.f;
  ln = wave_opaque(lane);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float e = __expf(z[j] - mxa);
    s_all += e;
    s_sel += ln + 64 * j >= S ? e : 0.f;
  }
  const float Z = wave_sum(s_all), Zs = wave_sum(s_sel);
  const float msum = S > 0 ? Zs / Z : 1.f;
  const float denom = fmaxf(msum, 1e-12f);
  if (probs_out) {
    const __amdgpu_buffer_rsrc_t ps = __builtin_amdgcn_make_buffer_rsrc(probs_out + r * C, (short)0, Ci * 4, 0x00020000);
#pragma unroll
    for (int j = 0; j < E; ++j)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, __expf(z[j] - mxa) / Z), ps, lane * 4, 256 * j, 0);
  }

  // ---- fast selection: t0 = the k-th largest of the 64 lanes' maxima; at least k selectable
  // logits are >= t0, so the top k are among them.  Those candidates (a few dozen for any spread
  // of values) are ranked exactly, which is also the final order.
  {
    int lrank = 0;
    for (int i = 0; i < 64; ++i) {
      const float m = __shfl(lane_hi, i, 64);
      lrank += (m > lane_hi) || (m == lane_hi && i < lane);
    }
    const uint64_t at = __ballot(lrank == k - 1);
    const float t0 = __shfl(lane_hi, __builtin_ctzll(at), 64);
    int ncand = 0;
    {
      const int ln0 = wave_opaque(lane);
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const int c = ln0 + 64 * j;
        const bool cand = c < Ci && c >= S && z[j] >= t0;
        const uint64_t mc = __ballot(cand);
        if (cand) {
          const int p = ncand + lanes_below(mc);
          if (p < kWaveCand) {
            sm.cand_key[p] = fkey(z[j]);
            sm.cand_idx[p] = c;
          }
        }
        ncand += __popcll(mc);
      }
    }
    if (ncand <= kWaveCand && t0 > -INFINITY) {
      wave_lds_sync();
      for (int i = lane; i < ncand; i += 64) {
        const uint32_t ki = sm.cand_key[i];
        const int32_t ii = sm.cand_idx[i];
        int rank = 0;
        for (int j = 0; j < ncand; ++j) {
          const uint32_t kj = sm.cand_key[j];
          rank += (kj > ki) || (kj == ki && sm.cand_idx[j] < ii);
        }
        if (rank < k) {
          float p = __expf(fkey_inv(ki) - mxa) / Z;
          if (S > 0) p = p / denom;
          sm.sorted_w[rank] = p;
          sm.sorted_i[rank] = ii;
        }
      }
      wave_lds_sync();
      const float ps = lane < k ? sm.sorted_w[lane] : 0.f;
      const float W = fmaxf(wave_sum(ps), 1e-12f);
      if (lane < k) {
        const float wn = ps / W;
        idx_out[r * k + lane] = sm.sorted_i[lane];
        w_out[r * k + lane] = wn;
        sm.sorted_w[lane] = wn;
      }
      if (!idx_star) return;
      wave_lds_sync();
      prepend_row(sm.sorted_i, sm.sorted_w, k, S, scale, idx_star + r * (S + k), omega + r * (S + k), lane);
      return;
    }
    wave_lds_sync();
  }

  // ---- selection into sm.sel_key / sm.sel_idx (any order)
  const float inv = (float)kWaveBins / (hi - lo);
  const bool binned = hi > lo && inv > 0.f && inv < INFINITY;
  auto bin_of = [&](float v) { return binned ? min(kWaveBins - 1, (int)((v - lo) * inv)) : 0; };
  wave_lds_sync();
  // boundary bin (every selectable logit in bin 0 when the range does not split)
  int bstar = 0, remaining = k, nb = Ci - S;
  if (binned) {
    ln = wave_opaque(lane);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int c = ln + 64 * j;
      const bool sel = c < Ci && c >= S;
      atomicAdd(&sm.hist[sel ? bin_of(z[j]) : 0], sel ? 1 : 0);
    }
    wave_lds_sync();
    constexpr int BPL = kWaveBins / 64;
    int cnt[BPL], mine = 0;
#pragma unroll
    for (int i = 0; i < BPL; ++i) {
      cnt[i] = sm.hist[lane * BPL + i];
      mine += cnt[i];
    }
    int above = wave_suffix_sum(mine, lane) - mine;
    int my_b = -1, my_rem = 0, my_nb = 0;
#pragma unroll
    for (int i = BPL - 1; i >= 0; --i) {
      if (above < k && above + cnt[i] >= k) {
        my_b = lane * BPL + i;
        my_rem = k - above;
        my_nb = cnt[i];
      }
      above += cnt[i];
    }
    const int src = __builtin_ctzll(__ballot(my_b >= 0));
    bstar = __shfl(my_b, src, 64);
    remaining = __shfl(my_rem, src, 64);
    nb = __shfl(my_nb, src, 64);
  }
  const int n_above = k - remaining;
  const bool direct = nb <= kWaveCand;
  // logits above the boundary bin are selected, the boundary bin's are candidates (slots taken
  // from per-wave LDS counters; the order is fixed by the ranks below).  The bins are formed
  // again here rather than kept from the histogram pass (72 more live registers).
  ln = wave_opaque(lane);
  float lo2 = lo, inv2 = inv;
  asm volatile("" : "+v"(lo2), "+v"(inv2));
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int c = ln + 64 * j;
    const int b = binned ? min(kWaveBins - 1, (int)((z[j] - lo2) * inv2)) : 0;
    if (c < Ci && c >= S && b >= bstar) {
      if (b > bstar) {
        const int p = atomicAdd(&sm.count[0], 1);
        sm.sel_key[p] = fkey(z[j]);
        sm.sel_idx[p] = c;
      } else if (direct) {
        const int p = atomicAdd(&sm.count[1], 1);
        sm.cand_key[p] = fkey(z[j]);
        sm.cand_idx[p] = c;
      }
    }
  }
  wave_lds_sync();
  if (direct) {
    // the `remaining` best of the boundary bin
    for (int i = lane; i < nb; i += 64) {
      const uint32_t ki = sm.cand_key[i];
      const int32_t ii = sm.cand_idx[i];
      int rank = 0;
      for (int j = 0; j < nb; ++j) {
        const uint32_t kj = sm.cand_key[j];
        rank += (kj > ki) || (kj == ki && sm.cand_idx[j] < ii);
      }
      if (rank < remaining) {
        sm.sel_key[n_above + rank] = ki;
        sm.sel_idx[n_above + rank] = ii;
      }
    }
  } else {
    // crowded boundary bin: one wave-wide maximum of (key, -id) per remaining slot; the pairs
    // taken are exactly those at or above the last one taken
    uint64_t last = ~0ull;
    for (int t = 0; t < remaining; ++t) {
      uint64_t best = 0;
      ln = wave_opaque(lane);
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const int c = ln + 64 * j;
        const uint64_t v = ((uint64_t)fkey(z[j]) << 32) | (uint32_t)~(uint32_t)c;
        const bool cand = c < Ci && c >= S && bin_of(z[j]) == bstar && v < last;
        best = cand && v > best ? v : best;
      }
      best = wave_max_u64(best);
      if (lane == 0) {
        sm.sel_key[n_above + t] = (uint32_t)(best >> 32);
        sm.sel_idx[n_above + t] = (int32_t)~(uint32_t)best;
      }
      last = best;
    }
  }
  wave_lds_sync();
  // ---- rank order (key descending, id ascending), probabilities, renormalisation in rank order
  if (lane < k) {
    const uint32_t ki = sm.sel_key[lane];
    const int32_t ii = sm.sel_idx[lane];
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const uint32_t kj = sm.sel_key[j];
      rank += (kj > ki) || (kj == ki && sm.sel_idx[j] < ii);
    }
    float p = __expf(fkey_inv(ki) - mxa) / Z;
    if (S > 0) p = p / denom;
    sm.sorted_w[rank] = p;
    sm.sorted_i[rank] = ii;
  }
  wave_lds_sync();
  const float ps = lane < k ? sm.sorted_w[lane] : 0.f;
  const float W = fmaxf(wave_sum(ps), 1e-12f);
  if (lane < k) {
    const float wn = ps / W;
    idx_out[r * k + lane] = sm.sorted_i[lane];
    w_out[r * k + lane] = wn;
    sm.sorted_w[lane] = wn;
  }
  if (!idx_star) return;
  wave_lds_sync();
  prepend_row(sm.sorted_i, sm.sorted_w, k, S, scale, idx_star + r * (S + k), omega + r * (S + k), lane);
}

// Backward of the top-k chain (router.py:114-149 autograd, as topk_bwd_row) within one wave per
// row.  With q = softmax(z), the masked renormalisation p' = q / D (D = clamp(sum_{c>=S} q)), the
// selected w_raw = p'[idx] and w = w_raw / clamp(sum w_raw): dq_c = base for every c >= S plus
// dw_raw_i / D at c = idx_i, base = -A / D^2 (A = sum_i dw_raw_i q[idx_i]), and
// sum_c dq_c q_c = base * msum + A / D (msum = sum_{c>=S} q), so dz = q (dq - that) needs no dense
// dq: the row is stored with dq = base, then the k selected entries are rewritten.
template <int E>
__global__ __launch_bounds__(64 * kWaveRows) void router_topk_bwd_wave_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ idx, const float* __restrict__ dw_hat, int64_t R,
    int64_t C, int S, int k, const float* __restrict__ dz_in, float* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r = (int64_t)blockIdx.x * kWaveRows + wv;  // wave-uniform: the row's buffer resources stay scalar
  if (r >= R) return;
  const float* row = logits + r * C;
  int32_t ci = 0;
  float g = 0.f, zi = 0.f;
  if (lane < k) {
    ci = idx[r * k + lane];
    g = dw_hat[r * k + lane];
    zi = row[ci];
  }
  const int Ci = (int)C;
  float z[E];
  wave_load_row(row, Ci, lane, z);
  float mxa = -INFINITY;
#pragma unroll
  for (int j = 0; j < E; ++j) mxa = fmaxf(mxa, z[j]);
  mxa = wave_max(mxa);
  float s_all = 0.f, s_sel = 0.f;
  int ln = wave_opaque(lane);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float e = __expf(z[j] - mxa);  // 0 for the -inf padding
    s_all += e;
    s_sel += ln + 64 * j >= S ? e : 0.f;
  }
  const float Z = wave_sum(s_all), Zs = wave_sum(s_sel);
  const float msum = S > 0 ? Zs / Z : 1.f;
  const float denom = fmaxf(msum, 1e-12f);
  const bool denom_live = msum >= 1e-12f;
  const float qi = lane < k ? __expf(zi - mxa) / Z : 0.f;
  const float pi = S > 0 ? qi / denom : qi;
  const float Wsum = wave_sum(pi), GW = wave_sum(g * pi);
  const float W = fmaxf(Wsum, 1e-12f);
  const bool W_live = Wsum >= 1e-12f;
  const float dwr = lane < k ? g / W - (W_live ? GW / (W * W) : 0.f) : 0.f;
  const float A = wave_sum(dwr * qi);
  const float base = (S > 0 && denom_live) ? -A / (denom * denom) : 0.f;
  const float dsel = S > 0 ? dwr / denom : dwr;
  const float DPP = (S > 0 ? base * msum : 0.f) + wave_sum(dsel * qi);
  float* out = dlogits + r * C;
  // buffer stores: the row's resource bound drops the padding's stores
  const __amdgpu_buffer_rsrc_t os = __builtin_amdgcn_make_buffer_rsrc(out, (short)0, Ci * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t is =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(dz_in ? dz_in + r * C : out), (short)0,
                                        dz_in ? Ci * 4 : 0, 0x00020000);
  const float iz = 1.f / Z;
  ln = wave_opaque(lane);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int c = ln + 64 * j;
    const float q = __expf(z[j] - mxa) * iz;
    const float dq = (S > 0 && c >= S) ? base : 0.f;
    const float din = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(is, lane * 4, 256 * j, 0));
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, q * (dq - DPP) + din), os, lane * 4, 256 * j, 0);
  }
  // the selected entries, after the dense stores have completed
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane < k) {
    const float dq = (S > 0 && ci >= S ? base : 0.f) + dsel;
    out[ci] = qi * (dq - DPP) + (dz_in ? dz_in[r * C + ci] : 0.f);
  }
}

// The same backward with the logit gradient consumed on the spot by the per-token router's
// backward products (router.py:294): instead of dlogits f32 [R, C] the kernel writes its bf16
// copy dzp [R, Cp] (columns C .. Cp-1 zero: the operand of dx = dz W and dW = dz^T x on the
// chapter kernels) and per-workgroup column sums of the fp32 values for the bias gradient.  A
// wave takes kPackWaveRows consecutive rows; its column sums stay in registers (lane l: columns
// l + 64 j) and the k selected entries' corrections go to the wave's LDS row; the workgroup's
// waves are added in wave order into one partial row.  The values are those of
// router_topk_bwd_wave_kernel (same expressions, same order).
constexpr int kPackWaveRows = 4;

template <bool DIN, int E>
__global__ __launch_bounds__(64 * kWaveRows) void router_topk_bwd_pack_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ idx, const float* __restrict__ dw_hat, int64_t R,
    int64_t C, int S, int k, const float* __restrict__ dz_in, int64_t Cp, bf16* __restrict__ dzp,
    float* __restrict__ part) {
  __shared__ float fix_all[kWaveRows][64 * E];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* fix = fix_all[wv];
  const int Ci = (int)C, Cpi = (int)Cp;
  float col[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    col[j] = 0.f;
    fix[lane + 64 * j] = 0.f;
  }
  const int64_t r0 = ((int64_t)blockIdx.x * kWaveRows + wv) * kPackWaveRows;
  for (int rr = 0; rr < kPackWaveRows; ++rr) {
    const int64_t r = r0 + rr;   // wave-uniform
    if (r >= R) break;
    const float* row = logits + r * C;
    int32_t ci = 0;
    float g = 0.f, zi = 0.f;
    if (lane < k) {
      ci = idx[r * k + lane];
      g = dw_hat[r * k + lane];
      zi = row[ci];
    }
    float z[E];
    wave_load_row(row, Ci, lane, z);
    float mxa = -INFINITY;
#pragma unroll
    for (int j = 0; j < E; ++j) mxa = fmaxf(mxa, z[j]);
    mxa = wave_max(mxa);
    float s_all = 0.f, s_sel = 0.f;
    int ln = wave_opaque(lane);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const float e = __expf(z[j] - mxa);
      s_all += e;
      s_sel += ln + 64 * j >= S ? e : 0.f;
    }
    const float Z = wave_sum(s_all), Zs = wave_sum(s_sel);
    const float msum = S > 0 ? Zs / Z : 1.f;
    const float denom = fmaxf(msum, 1e-12f);
    const bool denom_live = msum >= 1e-12f;
    const float qi = lane < k ? __expf(zi - mxa) / Z : 0.f;
    const float pi = S > 0 ? qi / denom : qi;
    const float Wsum = wave_sum(pi), GW = wave_sum(g * pi);
    const float W = fmaxf(Wsum, 1e-12f);
    const bool W_live = Wsum >= 1e-12f;
    const float dwr = lane < k ? g / W - (W_live ? GW / (W * W) : 0.f) : 0.f;
    const float A = wave_sum(dwr * qi);
    const float base = (S > 0 && denom_live) ? -A / (denom * denom) : 0.f;
    const float dsel = S > 0 ? dwr / denom : dwr;
    const float DPP = (S > 0 ? base * msum : 0.f) + wave_sum(dsel * qi);
    // bf16 row, the padding columns C .. Cp-1 included (their stores hold zeros)
    const __amdgpu_buffer_rsrc_t os = __builtin_amdgcn_make_buffer_rsrc(dzp + r * Cp, (short)0, Cpi * 2, 0x00020000);
    const float iz = 1.f / Z;
    ln = wave_opaque(lane);
    // with an incoming gradient, its row is read eight columns at a time ahead of their stores
    constexpr int kChunk = DIN ? 8 : E;
#pragma unroll
    for (int j0 = 0; j0 < E; j0 += kChunk) {
      float din[kChunk];
#pragma unroll
      for (int jj = 0; jj < kChunk; ++jj) {
        din[jj] = 0.f;
        if constexpr (DIN) {
          const __amdgpu_buffer_rsrc_t is =
              __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(dz_in + r * C), (short)0, Ci * 4, 0x00020000);
          din[jj] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(is, lane * 4, 256 * (j0 + jj), 0));
        }
      }
#pragma unroll
      for (int jj = 0; jj < kChunk; ++jj) {
        const int j = j0 + jj;
        const int c = ln + 64 * j;
        const float q = __expf(z[j] - mxa) * iz;
        const float dq = (S > 0 && c >= S) ? base : 0.f;
        const float v = q * (dq - DPP) + din[jj];   // 0 past C (q = 0 there, din reads zero)
        col[j] += v;
        const bf16 h = (bf16)v;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, h), os, lane * 2, 128 * j, 0);
      }
    }
    // the selected entries, after the dense stores have completed: their exact values, and the
    // difference to the dense value (q (dsel) ... ) into the wave's correction row
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane < k) {
      const float dq = (S > 0 && ci >= S ? base : 0.f) + dsel;
      const float din = DIN ? dz_in[r * C + ci] : 0.f;
      const float v = qi * (dq - DPP) + din;
      const float vd = qi * ((S > 0 && ci >= S ? base : 0.f) - DPP) + din;
      dzp[r * Cp + ci] = (bf16)v;
      fix[ci] += v - vd;   // distinct columns within a row: no two lanes touch one entry
    }
  }
  // this wave's column sums into its LDS row, then the workgroup's rows in wave order
#pragma unroll
  for (int j = 0; j < E; ++j) fix[lane + 64 * j] += col[j];
  __syncthreads();
  float* out = part + (int64_t)blockIdx.x * C;
  for (int c = threadIdx.x; c < Ci; c += 64 * kWaveRows) {
    float t = fix_all[0][c];
#pragma unroll
    for (int w = 1; w < kWaveRows; ++w) t += fix_all[w][c];
    out[c] = t;
  }
}

// Whether the one-wave-per-row kernels take these rows: many rows (the workgroup-per-row
// kernels suit a few long-latency rows better), short enough for registers, k <= 64.
inline bool router_wave_rows(int64_t R, int64_t C, int k) {
  return R > 64 && C <= 64 * kWaveMaxE && k <= kWaveMaxK;
}

// dlogits for the chain  p = softmax(z); q = p masked to c >= S; p' = q / clamp(sum q);
// w = p'[idx]; w_hat = w / clamp(sum w).  dw_hat is the incoming gradient (global or LDS).
// Mirrors autograd of memory_transformer/router.py:114-149 including the clamp_min(1e-12)
// gates.  The row (zs) and the dense dp vector (dps) live in LDS; dz_in (optional) is a
// gradient arriving at the logits from elsewhere (the router losses), added at the end.
template <int NT>
__device__ void topk_bwd_row(const float* zs, float* dps, int64_t C, int S, int k, const int32_t* __restrict__ idx,
                             const float* dw_hat, const float* __restrict__ dz_in, float* __restrict__ dz,
                             float* red, float* s_dwraw) {
  const int tid = threadIdx.x;
  const RowStats st = row_stats<NT>(zs, C, S, red);
  const float denom = fmaxf(st.msum, 1e-12f);
  const bool denom_live = st.msum >= 1e-12f;

  // w_raw and its sum
  float part = 0.f, gw = 0.f;
  for (int i = tid; i < k; i += NT) {
    float p = __expf(zs[idx[i]] - st.mx) / st.Z;
    if (S > 0) p = p / denom;
    part += p;
    gw += dw_hat[i] * p;
  }
  const float Wsum = block_reduce_sum<NT>(part, red);
  const float GW = block_reduce_sum<NT>(gw, red);  // sum_j g_j w_raw_j
  const float W = fmaxf(Wsum, 1e-12f);
  const bool W_live = Wsum >= 1e-12f;
  // dw_raw_i = g_i / W - [live] * GW / W^2 ; A = sum_i dw_raw_i * q_{idx_i}
  float a = 0.f;
  for (int i = tid; i < k; i += NT) {
    const float dwr = dw_hat[i] / W - (W_live ? GW / (W * W) : 0.f);
    s_dwraw[i] = dwr;
    const float p = __expf(zs[idx[i]] - st.mx) / st.Z;
    a += dwr * p;
  }
  const float A = block_reduce_sum<NT>(a, red);
  // dp_c: the mask/renormalisation term for every c >= S, plus the selected entries
  const float base = (S > 0 && denom_live) ? -A / (denom * denom) : 0.f;
  for (int64_t c = tid; c < C; c += NT) dps[c] = (S > 0 && c >= S) ? base : 0.f;
  __syncthreads();
  for (int i = tid; i < k; i += NT) dps[idx[i]] += (S > 0) ? s_dwraw[i] / denom : s_dwraw[i];
  __syncthreads();
  float dpp = 0.f;
  for (int64_t c = tid; c < C; c += NT) dpp += dps[c] * (__expf(zs[c] - st.mx) / st.Z);
  const float DPP = block_reduce_sum<NT>(dpp, red);
  for (int64_t c = tid; c < C; c += NT) {
    const float p = __expf(zs[c] - st.mx) / st.Z;
    dz[c] = p * (dps[c] - DPP) + (dz_in ? dz_in[c] : 0.f);
  }
}

template <int NT>
__global__ __launch_bounds__(NT) void router_topk_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ idx, const float* __restrict__ dw_hat,
    int64_t C, int S, int k, float* __restrict__ dlogits) {
  extern __shared__ float zs[];  // row [C] then dp [C]
  __shared__ float red[NT / 64];
  __shared__ float s_dwraw[kMaxTopK];
  const int64_t r = blockIdx.x;
  load_row<NT>(logits + r * C, C, zs);
  topk_bwd_row<NT>(zs, zs + C, C, S, k, idx + r * k, dw_hat + r * k, nullptr, dlogits + r * C, red, s_dwraw);
}

// The sequence router's backward from the attention's d omega to the logits, one workgroup
// per row: d omega_j = sum over kv heads of dom_part[(r NS + j) HK + hk] (NS = S + k slots),
// the prepend's backward (prepend_row_bwd) to dw, the top-k chain's backward (topk_bwd_row),
// plus dz_in.  w is the top-k's output weights (the prepend's input).
template <int NT>
__global__ __launch_bounds__(NT) void router_seq_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ idx, const float* __restrict__ w,
    const float* __restrict__ dom_part, int HK, int64_t C, int S, int k, float scale,
    const float* __restrict__ dz_in, float* __restrict__ dlogits) {
  extern __shared__ float zs[];  // row [C] then dp [C]
  __shared__ float red[NT / 64];
  __shared__ float s_dwraw[kMaxTopK];
  __shared__ float s_dom[kMaxTopK + kMaxSeqShared];
  __shared__ float s_dw[kMaxTopK];
  const int64_t r = blockIdx.x;
  const int NS = S + k;
  const int tid = threadIdx.x;
  for (int j = tid; j < NS; j += NT) {
    const float* p = dom_part + ((int64_t)r * NS + j) * HK;
    float t = 0.f;
    for (int h = 0; h < HK; ++h) t += p[h];
    s_dom[j] = t;
  }
  load_row<NT>(logits + r * C, C, zs);  // (ends with a barrier)
  if (tid < 64) prepend_row_bwd(w + r * k, s_dom, k, S, scale, s_dw, tid);
  __syncthreads();
  topk_bwd_row<NT>(zs, zs + C, C, S, k, idx + r * k, s_dw, dz_in ? dz_in + r * C : nullptr, dlogits + r * C, red,
                   s_dwraw);
}

// omega = [1..1 (S), scale * w] / clamp(sum); idx_star = [0..S-1, idx]; one wave per row.
__global__ void prepend_kernel(const int32_t* __restrict__ idx, const float* __restrict__ w, int64_t R,
                               int k, int S, float scale, int32_t* __restrict__ idx_star,
                               float* __restrict__ omega) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (r >= R) return;
  prepend_row(idx + r * k, w + r * k, k, S, scale, idx_star + r * (S + k), omega + r * (S + k), threadIdx.x);
}

__global__ void prepend_bwd_kernel(const float* __restrict__ w, const float* __restrict__ domega, int64_t R,
                                   int k, int S, float scale, float* __restrict__ dw) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (r >= R) return;
  prepend_row_bwd(w + r * k, domega + r * (S + k), k, S, scale, dw + r * k, threadIdx.x);
}

// pooled[b, :] = sum_l coef[l] * h[b, l, :]   (coef == nullptr: mean over L).
// grid (B, nsplit), 128 threads: thread t sums 8-column chunks t, t + 128, ... of
// rows [l0, l1) with several 16/32-byte loads in flight; partials [nsplit][B][d]
// are reduced by pool_reduce.  d % 8 == 0 and 32-byte aligned rows (else pool_partial_cols).
constexpr int kPoolThreads = 128;
template <typename T>
__global__ __launch_bounds__(kPoolThreads) void pool_partial_kernel(const T* __restrict__ h, int64_t L, int64_t d,
                                                                    const float* __restrict__ coef,
                                                                    int rows_per_split, float* __restrict__ part) {
  const int64_t b = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t l0 = (int64_t)split * rows_per_split;
  const int64_t l1 = min((int64_t)L, l0 + rows_per_split);
  for (int64_t c8 = (int64_t)threadIdx.x * 8; c8 < d; c8 += kPoolThreads * 8) {
    const T* hb = h + b * L * d + c8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t l = l0;
    for (; l + 4 <= l1; l += 4) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) ChunkLoadF<T>::run(hb + (l + u) * d, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float cw = coef ? coef[l + u] : 1.f;
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[x] += cw * v[u][x];
      }
    }
    for (; l < l1; ++l) {
      float v[8];
      ChunkLoadF<T>::run(hb + l * d, v);
      const float cw = coef ? coef[l] : 1.f;
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] += cw * v[x];
    }
    float* dst = part + ((int64_t)split * gridDim.x + b) * d + c8;
    *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  }
}

// pool_partial for any d (rows need not be 16-byte aligned): thread t sums single
// columns t, t + 128, ... with coalesced 4-byte loads, 8 rows in flight.
template <typename T>
__global__ __launch_bounds__(kPoolThreads) void pool_partial_cols_kernel(const T* __restrict__ h, int64_t L,
                                                                         int64_t d, const float* __restrict__ coef,
                                                                         int rows_per_split, float* __restrict__ part) {
  const int64_t b = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t l0 = (int64_t)split * rows_per_split;
  const int64_t l1 = min((int64_t)L, l0 + rows_per_split);
  for (int64_t c = threadIdx.x; c < d; c += kPoolThreads) {
    const T* hb = h + b * L * d + c;
    float acc = 0.f;
    int64_t l = l0;
    for (; l + 8 <= l1; l += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = to_f(hb[(l + u) * d]);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += (coef ? coef[l + u] : 1.f) * v[u];
    }
    for (; l < l1; ++l) acc += (coef ? coef[l] : 1.f) * to_f(hb[l * d]);
    part[((int64_t)split * gridDim.x + b) * d + c] = acc;
  }
}

// One-launch pooling for 16-byte rows: pooled[b, c] = scale * sum_l coef[l] h[b, l, c]
// (coef == nullptr: scale = 1 / L).  Workgroup (b, 64-column block), 1,024 threads: thread t sums
// 8 columns (chunk t % 8) over the rows l = t / 8 (mod 128) with up to eight 16-byte loads in
// flight, so L <= 1,024 rows are read in one round; the 128 row groups are added in a fixed
// order through LDS (16 groups per thread, then 8 sums).  d % 8 == 0, rows 16-byte aligned.
constexpr int kPool1Groups = 128;
template <typename T>
__global__ __launch_bounds__(1024) void pool_single_kernel(const T* __restrict__ h, int64_t L, int64_t d,
                                                           const float* __restrict__ coef, float scale,
                                                           float* __restrict__ pooled) {
  __shared__ float part[kPool1Groups][65];
  __shared__ float part2[8][65];
  const int64_t b = blockIdx.y;
  const int chunk = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const int64_t c8 = (int64_t)blockIdx.x * 64 + 8 * chunk;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c8 < d) {
    const T* hb = h + b * L * d + c8;
    int64_t l = grp;
    for (; l + 7 * kPool1Groups < L; l += 8 * kPool1Groups) {
      float v[8][8];
#pragma unroll
      for (int u = 0; u < 8; ++u) ChunkLoadF<T>::run(hb + (l + u * kPool1Groups) * d, v[u]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float cw = coef ? coef[l + u * kPool1Groups] : 1.f;
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[x] += cw * v[u][x];
      }
    }
    for (; l < L; l += kPool1Groups) {
      float v[8];
      ChunkLoadF<T>::run(hb + l * d, v);
      const float cw = coef ? coef[l] : 1.f;
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] += cw * v[x];
    }
  }
#pragma unroll
  for (int x = 0; x < 8; ++x) part[grp][8 * chunk + x] = acc[x];
  __syncthreads();
  if (threadIdx.x < 512) {
    const int col = threadIdx.x & 63, q = threadIdx.x >> 6;
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) t += part[16 * q + g][col];
    part2[q][col] = t;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int64_t c = (int64_t)blockIdx.x * 64 + threadIdx.x;
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) t += part2[q][threadIdx.x];
    if (c < d) pooled[b * d + c] = t * scale;
  }
}

// x[b, l, :] += v[b, :] * (coef ? coef[l] : scale), in place (the pooling's backward added into
// a gradient that already holds another contribution).  One thread per 8 columns of a row.
template <typename T>
__global__ __launch_bounds__(256) void rows_add_bcast_kernel(T* __restrict__ x, int64_t B, int64_t L, int64_t d,
                                                             const float* __restrict__ v,
                                                             const float* __restrict__ coef, float scale) {
  const int64_t n8 = d / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= B * L * n8) return;
  const int64_t row = i / n8, c8 = (i - row * n8) * 8;
  const int64_t b = row / L, l = row - b * L;
  const float cw = coef ? coef[l] : scale;
  T* p = x + row * d + c8;
  float a[8];
  ChunkLoadF<T>::run(p, a);
  const f32x4 v0 = *reinterpret_cast<const f32x4*>(v + b * d + c8);
  const f32x4 v1 = *reinterpret_cast<const f32x4*>(v + b * d + c8 + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] += cw * v0[e];
    a[4 + e] += cw * v1[e];
  }
  if constexpr (sizeof(T) == 2) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)a[e];
    *reinterpret_cast<bf16x8*>(p) = o;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{a[0], a[1], a[2], a[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{a[4], a[5], a[6], a[7]};
  }
}

// out[i] = inv * sum_j part[j][i] for i < n, j < nsplit.  A workgroup owns 64
// consecutive outputs; its 4 waves sum interleaved quarters of the partials with
// 8 loads in flight, then wave 0 adds the 4 quarters in order (deterministic).
__global__ __launch_bounds__(256) void pool_reduce_kernel(const float* __restrict__ part, int nsplit, int64_t B,
                                                          int64_t d, float inv, float* __restrict__ out) {
  __shared__ float q4[4][64];
  const int64_t n = B * d;
  const int o = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + o;
  float s = 0.f;
  if (i < n) {
    // 32 loads in flight per thread before the first add (a reduction over a few hundred splits
    // is then two or three rounds of memory latency, not one per eight loads: it often runs on
    // the few CUs other kernels leave free)
    int j = g;
    for (; j + 124 < nsplit; j += 128) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) v[u] = part[(int64_t)(j + 4 * u) * n + i];
#pragma unroll
      for (int u = 0; u < 32; ++u) s += v[u];
    }
    if (j < nsplit) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) v[u] = j + 4 * u < nsplit ? part[(int64_t)(j + 4 * u) * n + i] : 0.f;
#pragma unroll
      for (int u = 0; u < 32; ++u) s += v[u];
    }
  }
  q4[g][o] = s;
  __syncthreads();
  if (g == 0 && i < n) out[i] = (q4[0][o] + q4[1][o] + q4[2][o] + q4[3][o]) * inv;
}

// Router linear for few rows (one per sequence).  A workgroup owns kLinChap
// consecutive chapters (4 per wave) and stages up to kLinRows rows of x in LDS,
// so W is streamed from HBM once and x is read from LDS.  Every loop keeps its
// global loads in registers before the first use (4 floats per lane per load),
// so a thread never waits on one load at a time.  d % 4 == 0.
constexpr int kLinChap = 16;
constexpr int kLinRows = 16;
// The forward gives each wave one chapter (4 per workgroup): its cost is the per-(chapter, row)
// wave reductions, so more, smaller workgroups keep more of them in flight.
constexpr int kLinCpw = 1;
constexpr int kLinChapFwd = 4 * kLinCpw;

__device__ __forceinline__ f32x4 load4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 load4f(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

// xs[0 .. n) = x[0 .. n), n % 4 == 0, 16-byte loads, 4 in flight per thread
__device__ __forceinline__ void stage_rows(const float* __restrict__ x, int64_t n, float* xs) {
  int64_t i = (int64_t)threadIdx.x * 4;
  for (; i + 3 * 1024 < n; i += 4 * 1024) {
    const f32x4 a = load4f(x + i), b = load4f(x + i + 1024), c = load4f(x + i + 2048), e = load4f(x + i + 3072);
    *reinterpret_cast<f32x4*>(xs + i) = a;
    *reinterpret_cast<f32x4*>(xs + i + 1024) = b;
    *reinterpret_cast<f32x4*>(xs + i + 2048) = c;
    *reinterpret_cast<f32x4*>(xs + i + 3072) = e;
  }
  for (; i < n; i += 1024) *reinterpret_cast<f32x4*>(xs + i) = load4f(x + i);
}

template <typename TW>
__global__ __launch_bounds__(256) void router_linear_kernel(const float* __restrict__ x, int64_t R, int64_t d,
                                                            const TW* __restrict__ W, const float* __restrict__ bias,
                                                            int64_t C, float* __restrict__ logits) {
  extern __shared__ float xs[];  // [min(R, kLinRows)][d]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t c0 = (int64_t)blockIdx.x * kLinChapFwd + kLinCpw * wave;  // this wave's chapters
  // the first kLinPre 256-column chunks of the wave's W rows are loaded before x is staged (the
  // two load latencies overlap) and kept for every chunk of rows; wider rows stream the rest
  constexpr int kLinPre = 4;
  f32x4 wpre[kLinPre][kLinCpw];
#pragma unroll
  for (int i = 0; i < kLinPre; ++i)
#pragma unroll
    for (int q = 0; q < kLinCpw; ++q) {
      const int64_t j = 4 * lane + 256 * i;
      wpre[i][q] = (c0 + q < C && j < d) ? load4f(W + (c0 + q) * d + j) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  for (int64_t r0 = 0; r0 < R; r0 += kLinRows) {
    const int nr = (int)min((int64_t)kLinRows, R - r0);
    __syncthreads();
    stage_rows(x + r0 * d, (int64_t)nr * d, xs);
    __syncthreads();
    float acc[kLinCpw][kLinRows];
#pragma unroll
    for (int q = 0; q < kLinCpw; ++q)
#pragma unroll
      for (int r = 0; r < kLinRows; ++r) acc[q][r] = 0.f;
#pragma unroll
    for (int i = 0; i < kLinPre; ++i) {
      const int64_t j = 4 * lane + 256 * i;
      if (j < d) {
#pragma unroll
        for (int r = 0; r < kLinRows; ++r) {
          if (r < nr) {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + r * d + j);
#pragma unroll
            for (int q = 0; q < kLinCpw; ++q)
              acc[q][r] += xv[0] * wpre[i][q][0] + xv[1] * wpre[i][q][1] + xv[2] * wpre[i][q][2] +
                           xv[3] * wpre[i][q][3];
          }
        }
      }
    }
    for (int64_t j = 4 * lane + 256 * kLinPre; j < d; j += 256) {
      f32x4 wv[kLinCpw];
#pragma unroll
      for (int q = 0; q < kLinCpw; ++q)
        wv[q] = c0 + q < C ? load4f(W + (c0 + q) * d + j) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < kLinRows; ++r) {
        if (r < nr) {  // (a guard, not a break: the loop must unroll fully to keep acc in registers)
          const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + r * d + j);
#pragma unroll
          for (int q = 0; q < kLinCpw; ++q)
            acc[q][r] += xv[0] * wv[q][0] + xv[1] * wv[q][1] + xv[2] * wv[q][2] + xv[3] * wv[q][3];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kLinCpw; ++q) {
      const int64_t c = c0 + q;
      const float bc = (bias && c < C) ? bias[c] : 0.f;
#pragma unroll
      for (int r = 0; r < kLinRows; ++r) {
        if (r < nr) {
          const float v = wave_sum(acc[q][r]);
          if (lane == 0 && c < C) logits[(r0 + r) * C + c] = v + bc;
        }
      }
    }
  }
}

// Router linear for few rows on the fp32 matrix cores (v_mfma_f32_16x16x4_f32): a workgroup owns
// 16 chapters; its 4 waves split d into quarters (d % 64 == 0) and hold every W and x chunk of
// their quarter in registers before the first product (one round of loads); the 4 partial
// 16 x 16 tiles (chapters x rows) are added in wave order through LDS.  Lane (m, g) of an MFMA
// k-block of 16 columns supplies W[c0 + m][kb + 4g + j] and x[r0 + m][kb + 4g + j] for step j,
// so both operands are 16-byte loads.  Rows are taken 16 at a time.
template <typename TW, int KB>
__global__ __launch_bounds__(256) void router_linear_mfma_kernel(const float* __restrict__ x, int64_t R, int64_t d,
                                                                 const TW* __restrict__ W,
                                                                 const float* __restrict__ bias, int64_t C,
                                                                 float* __restrict__ logits) {
  __shared__ f32x4 red[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = lane & 15, g = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 16;
  const int64_t kq = d / 4, k0 = wave * kq;  // this wave's quarter of d
  const int nkb = (int)(kq / 16);
  // W chunks of this wave's quarter (KB blocks kept in registers; wider rows stream the rest)
  f32x4 wreg[KB];
  const bool crow = c0 + m < C;
#pragma unroll
  for (int i = 0; i < KB; ++i)
    wreg[i] = (crow && i < nkb) ? load4f(W + (c0 + m) * d + k0 + 16 * i + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t r0 = 0; r0 < R; r0 += 16) {
    const bool rrow = r0 + m < R;
    f32x4 xreg[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i)
      xreg[i] = (rrow && i < nkb) ? load4f(x + (r0 + m) * d + k0 + 16 * i + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wreg[i][j], xreg[i][j], acc, 0, 0, 0);
    for (int i = KB; i < nkb; ++i) {
      const f32x4 wv = crow ? load4f(W + (c0 + m) * d + k0 + 16 * i + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 xv = rrow ? load4f(x + (r0 + m) * d + k0 + 16 * i + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[j], xv[j], acc, 0, 0, 0);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      // lane (n = row, g) holds chapters 4g + e of row n
      const f32x4 t = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
      const int64_t r = r0 + m;
      if (r < R) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t c = c0 + 4 * g + e;
          if (c < C) logits[r * C + c] = t[e] + (bias ? bias[c] : 0.f);
        }
      }
    }
    __syncthreads();
  }
}

// Backward of the router linear for few rows, one pass over W:
//   dW[c, :] = sum_r dz[r, c] x[r, :],  db[c] = sum_r dz[r, c]   (workgroup's chapters)
//   part[wg][r][j] = sum_{c of wg} dz[r, c] W[c, j]               (dx partial, 4 columns per thread)
// the dx partials are summed over workgroups by pool_reduce (fixed order).
template <typename TW>
__global__ __launch_bounds__(256) void router_linear_bwd_kernel(const float* __restrict__ dz,
                                                                const float* __restrict__ x, int64_t R, int64_t d,
                                                                const TW* __restrict__ W, int64_t C,
                                                                float* __restrict__ dW, float* __restrict__ db,
                                                                float* __restrict__ part) {
  extern __shared__ float xs[];  // [kLinRows][d]
  __shared__ float dzs[kLinRows][kLinChap];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t cbase = (int64_t)blockIdx.x * kLinChap;
  const int nc = (int)min((int64_t)kLinChap, C - cbase);
  for (int64_t r0 = 0; r0 < R; r0 += kLinRows) {
    const int nr = (int)min((int64_t)kLinRows, R - r0);
    __syncthreads();
    if (dW) stage_rows(x + r0 * d, (int64_t)nr * d, xs);
    {
      const int r = threadIdx.x / kLinChap, cc = threadIdx.x % kLinChap;  // 256 = 16 x 16
      dzs[r][cc] = (r < nr && cc < nc) ? dz[(r0 + r) * C + cbase + cc] : 0.f;
    }
    __syncthreads();
    // dW rows of this wave's 4 chapters (x from LDS, no global loads in the loop)
    if (dW) {
      for (int q = 0; q < 4; ++q) {
        const int cc = 4 * wave + q;
        if (cc >= nc) break;
        float* dst = dW + (cbase + cc) * d;
        for (int64_t j = 4 * lane; j < d; j += 256) {
          f32x4 a = r0 > 0 ? *reinterpret_cast<const f32x4*>(dst + j) : f32x4{0.f, 0.f, 0.f, 0.f};
          for (int r = 0; r < nr; ++r) a += dzs[r][cc] * *reinterpret_cast<const f32x4*>(xs + r * d + j);
          *reinterpret_cast<f32x4*>(dst + j) = a;
        }
      }
    }
    if (db && threadIdx.x < nc) {
      float sacc = r0 > 0 ? db[cbase + threadIdx.x] : 0.f;
      for (int r = 0; r < nr; ++r) sacc += dzs[r][threadIdx.x];
      db[cbase + threadIdx.x] = sacc;
    }
    if (part) {
      for (int64_t j = 4 * (int64_t)threadIdx.x; j < d; j += 1024) {
        f32x4 wv[kLinChap];
#pragma unroll
        for (int cc = 0; cc < kLinChap; ++cc) wv[cc] = cc < nc ? load4f(W + (cbase + cc) * d + j) : f32x4{0.f, 0.f, 0.f, 0.f};
        for (int r = 0; r < nr; ++r) {
          f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int cc = 0; cc < kLinChap; ++cc) a += dzs[r][cc] * wv[cc];
          *reinterpret_cast<f32x4*>(part + ((int64_t)blockIdx.x * R + r0 + r) * d + j) = a;
        }
      }
    }
  }
}

// ------------------------------------------------------------ router auxiliary losses
// ChapterRouter._compute_losses (router.py:197-260) on logits z [R][C] and the selected
// chapter ids I [R][k], p = softmax(z) per row:
//   load_balance = C sum_c f_c P_c,  f_c = counts_c / R (selections of c),  P_c = mean_r p_rc
//   auxiliary    = mean_c (Q_c - 1/C)^2,  Q_c = mean_r p_rc^2   (F.mse_loss)
//   z_loss       = mean_r lse_r^2,  lse_r = log sum_c exp z_rc
//   entropy      = -mean_r sum_c p_rc log(max(p_rc, 1e-12))
// Row statistics one wave per row (lse, entropy; the row's selections counted by exact
// integer atomics), the column sums of p and p^2 one thread per column over a slice of rows
// (coalesced; partials reduced in a fixed order by pool_reduce), then one workgroup for the
// four scalars.  The backward is one wave per row.
constexpr int kLossThreads = 256;
constexpr int kLossColRows = 128;          // rows per column-sum workgroup
constexpr int kLossFinalThreads = 1024;

__global__ __launch_bounds__(kLossThreads) void router_loss_zero_kernel(int32_t* __restrict__ counts, int64_t C) {
  const int64_t c = (int64_t)blockIdx.x * kLossThreads + threadIdx.x;
  if (c < C) counts[c] = 0;
}

// log(1e-12): the floor the entropy term's clamp puts under log p
constexpr float kLogPFloor = -27.631021115928547f;
// Rows of up to kLossThreads * kLossRowCols chapters are held in registers by one workgroup
// (one read of the logits, all loads in flight at once); longer rows are streamed by one
// wave each.
constexpr int kLossRowCols = 18;

// Streamed: one wave per row, three passes over the row.
__global__ __launch_bounds__(kLossThreads) void router_loss_rowstats_kernel(
    const float* __restrict__ z, int64_t R, int64_t C, const int32_t* __restrict__ idx, int k,
    float* __restrict__ row_lse, float* __restrict__ row_ent, int32_t* __restrict__ counts) {
  const int64_t r = (int64_t)blockIdx.x * (kLossThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= R) return;
  const float* zr = z + r * C;
  float m = -INFINITY;
  for (int64_t c = lane; c < C; c += 64) m = fmaxf(m, zr[c]);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t c = lane; c < C; c += 64) s += __expf(zr[c] - m);
  const float lse = m + __logf(wave_sum(s));
  float e = 0.f;
  for (int64_t c = lane; c < C; c += 64) {
    const float lz = zr[c] - lse;
    e += __expf(lz) * fmaxf(lz, kLogPFloor);
  }
  e = wave_sum(e);
  if (lane == 0) {
    row_lse[r] = lse;
    row_ent[r] = e;
  }
  for (int j = lane; j < k; j += 64) {
    const int32_t c = idx[r * k + j];
    if (c >= 0 && c < C) atomicAdd(&counts[c], 1);   // integer: exact in any order
  }
}

// Register-resident: one workgroup per row (C <= kLossThreads * kLossRowCols).
// p log max(p, 1e-12) is taken with log p = z - lse (no log per element); past the row
// z = -inf, p = 0 and the term vanishes.
__global__ __launch_bounds__(kLossThreads) void router_loss_rowstats_block_kernel(
    const float* __restrict__ z, int64_t R, int64_t C, const int32_t* __restrict__ idx, int k,
    float* __restrict__ row_lse, float* __restrict__ row_ent, int32_t* __restrict__ counts) {
  __shared__ float red[kLossThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const float* zr = z + r * C;
  float v[kLossRowCols];
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) {
    const int64_t c = tid + kLossThreads * i;
    v[i] = c < C ? zr[c] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) m = fmaxf(m, v[i]);
  m = block_reduce_max<kLossThreads>(m, red);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) s += __expf(v[i] - m);
  const float lse = m + __logf(block_reduce_sum<kLossThreads>(s, red));
  float e = 0.f;
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) {
    const float lz = v[i] - lse;
    e += __expf(lz) * fmaxf(lz, kLogPFloor);
  }
  e = block_reduce_sum<kLossThreads>(e, red);
  if (tid == 0) {
    row_lse[r] = lse;
    row_ent[r] = e;
  }
  for (int j = tid; j < k; j += kLossThreads) {
    const int32_t c = idx[r * k + j];
    if (c >= 0 && c < C) atomicAdd(&counts[c], 1);
  }
}

// part[split][0][c] = sum over the split's rows of p_rc, part[split][1][c] of p_rc^2
__global__ __launch_bounds__(kLossThreads) void router_loss_colsum_kernel(const float* __restrict__ z, int64_t R,
                                                                          int64_t C,
                                                                          const float* __restrict__ row_lse,
                                                                          float* __restrict__ part) {
  const int64_t c = (int64_t)blockIdx.x * kLossThreads + threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * kLossColRows, r1 = min(R, r0 + kLossColRows);
  if (c >= C) return;
  float sp = 0.f, sq = 0.f;
  int64_t r = r0;
  for (; r + 4 <= r1; r += 4) {
    float p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p[u] = __expf(z[(r + u) * C + c] - row_lse[r + u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      sp += p[u];
      sq += p[u] * p[u];
    }
  }
  for (; r < r1; ++r) {
    const float p = __expf(z[r * C + c] - row_lse[r]);
    sp += p;
    sq += p * p;
  }
  float* dst = part + (int64_t)blockIdx.y * 2 * C;
  dst[c] = sp;
  dst[C + c] = sq;
}

// losses[4] = {load_balance, auxiliary, z_loss, entropy}; coef[c] = the column's terms of the
// backward's per-element gradient (before the incoming loss gradients scale them):
//   coef[c].x = C counts_c / R^2          (load balance, d/dp_rc)
//   coef[c].y = 4 (Q_c - 1/C) / (C R)     (auxiliary, d/dp_rc per unit p_rc; Q_c = mean_r p_rc^2)
__global__ __launch_bounds__(kLossFinalThreads) void router_loss_final_kernel(
    const float* __restrict__ col, const float* __restrict__ row_lse, const float* __restrict__ row_ent,
    const int32_t* __restrict__ counts, int64_t R, int64_t C, float* __restrict__ losses,
    float2* __restrict__ coef) {
  __shared__ float red[kLossFinalThreads / 64];
  const int tid = threadIdx.x;
  const float invC = 1.f / (float)C, invR = 1.f / (float)R;
  const float cLB = (float)C * invR * invR, cAux = 4.f * invC * invR;
  // loads batched kUnroll at a time (one workgroup: latency, not bandwidth, bounds this kernel)
  constexpr int kUnroll = 4;
  float lb = 0.f, aux = 0.f;
  for (int64_t c0 = tid; c0 < C; c0 += kUnroll * kLossFinalThreads) {
    float n[kUnroll], pc[kUnroll], qc[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = c0 + u * kLossFinalThreads;
      n[u] = c < C ? (float)counts[c] : 0.f;
      pc[u] = c < C ? col[c] : 0.f;
      qc[u] = c < C ? col[C + c] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = c0 + u * kLossFinalThreads;
      if (c < C) {
        lb += n[u] * pc[u];
        const float t = qc[u] * invR - invC;
        aux += t * t;
        coef[c] = make_float2(cLB * n[u], cAux * t);
      }
    }
  }
  lb = block_reduce_sum<kLossFinalThreads>(lb, red);
  aux = block_reduce_sum<kLossFinalThreads>(aux, red);
  float zl = 0.f, en = 0.f;
  for (int64_t r0 = tid; r0 < R; r0 += kUnroll * kLossFinalThreads) {
    float l[kUnroll], e[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t r = r0 + u * kLossFinalThreads;
      l[u] = r < R ? row_lse[r] : 0.f;
      e[u] = r < R ? row_ent[r] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      zl += l[u] * l[u];
      en += e[u];
    }
  }
  zl = block_reduce_sum<kLossFinalThreads>(zl, red);
  en = block_reduce_sum<kLossFinalThreads>(en, red);
  if (tid == 0) {
    losses[0] = (float)C * lb * invR * invR;
    losses[1] = aux * invC;
    losses[2] = zl * invR;
    losses[3] = -en * invR;
  }
}

// Backward: dz_rc = p_rc (g_rc - sum_c' p_rc' g_rc' + gz (2 / R) lse_r) with
//   g_rc = gLB coef_c.x + gaux coef_c.y p_rc - gent (log max(p_rc, 1e-12) + [p_rc > 1e-12]) / R
// (dlosses = {gLB, gaux, gz, gent} on the device; coef from router_loss_final_kernel;
// log p_rc = z_rc - lse_r).
struct LossGrad {
  const float2* coef;
  float gLB, gaux, cEnt, zc;
  __device__ LossGrad(const float2* cf, const float* dlosses, int64_t R, float lse) : coef(cf) {
    const float invR = 1.f / (float)R;
    gLB = dlosses[0];
    gaux = dlosses[1];
    zc = dlosses[2] * 2.f * invR * lse;
    cEnt = dlosses[3] * invR;
  }
  // g_rc from log p_rc and p_rc
  __device__ float operator()(int64_t c, float lz, float p) const {
    const float2 cf = coef[c];
    return gLB * cf.x + gaux * cf.y * p - cEnt * (lz > kLogPFloor ? lz + 1.f : kLogPFloor);
  }
};

// Streamed: one wave per row, two passes over the row.
__global__ __launch_bounds__(kLossThreads) void router_loss_bwd_kernel(
    const float* __restrict__ z, int64_t R, int64_t C, const float* __restrict__ row_lse,
    const float2* __restrict__ coef, const float* __restrict__ dlosses, float* __restrict__ dz) {
  const int64_t r = (int64_t)blockIdx.x * (kLossThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= R) return;
  const float* zr = z + r * C;
  const float lse = row_lse[r];
  const LossGrad g(coef, dlosses, R, lse);
  float s = 0.f;
  for (int64_t c = lane; c < C; c += 64) {
    const float lz = zr[c] - lse, p = __expf(lz);
    s += p * g(c, lz, p);
  }
  s = wave_sum(s);
  float* o = dz + r * C;
  for (int64_t c = lane; c < C; c += 64) {
    const float lz = zr[c] - lse, p = __expf(lz);
    o[c] = p * (g(c, lz, p) - s + g.zc);
  }
}

// Register-resident: one workgroup per row (C <= kLossThreads * kLossRowCols).
__global__ __launch_bounds__(kLossThreads) void router_loss_bwd_block_kernel(
    const float* __restrict__ z, int64_t R, int64_t C, const float* __restrict__ row_lse,
    const float2* __restrict__ coef, const float* __restrict__ dlosses, float* __restrict__ dz) {
  __shared__ float red[kLossThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const float* zr = z + r * C;
  const float lse = row_lse[r];
  const LossGrad g(coef, dlosses, R, lse);
  // p[i] = p_rc, pg[i] = p_rc g_rc (0 past the row)
  float p[kLossRowCols], pg[kLossRowCols];
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) {
    const int64_t c = tid + kLossThreads * i;
    p[i] = c < C ? zr[c] - lse : -INFINITY;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) {
    const int64_t c = tid + kLossThreads * i;
    const float lz = p[i];
    p[i] = __expf(lz);
    pg[i] = c < C ? p[i] * g(c, lz, p[i]) : 0.f;
    s += pg[i];
  }
  s = block_reduce_sum<kLossThreads>(s, red) - g.zc;
  float* o = dz + r * C;
#pragma unroll
  for (int i = 0; i < kLossRowCols; ++i) {
    const int64_t c = tid + kLossThreads * i;
    if (c < C) o[c] = pg[i] - p[i] * s;
  }
}

int launch_split_reduce(const float* part, int nsplit, int64_t n, float inv, float* out, hipStream_t stream) {
  if (n <= 0) return MOC_OK;
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, stream, part, nsplit,
                     (int64_t)1, n, inv, out);
  return check_launch("pool_reduce_kernel");
}


// ------------------------------------------------------- per-token router: logit gradient pack
// The bf16 operand of the token router's two backward products (dx = dz W, dW = dz^T x) and the
// bias gradient (db = column sums of dz, router.py:294's nn.Linear bias) from one read of the fp32
// logit gradient: dzp [R][Cp] bf16 (columns C .. Cp-1 zero, so that both products run over a
// multiple of 256 chapters) and per-row-block column partials, summed in a fixed order.
constexpr int kPackRows = 64;  // rows per workgroup (one partial row of column sums)

__global__ __launch_bounds__(256) void logit_grad_pack_kernel(const float* __restrict__ dz, int64_t R, int64_t C,
                                                              int64_t Cp, bf16* __restrict__ dzp,
                                                              float* __restrict__ part) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;  // columns c, c + 1
  const int64_t r0 = (int64_t)blockIdx.y * kPackRows;
  if (c >= Cp) return;
  const int64_t r1 = min(R, r0 + kPackRows);
  const bool in0 = c < C, in1 = c + 1 < C;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 8
  for (int64_t r = r0; r < r1; ++r) {
    const float* row = dz + r * C;
    const float a = in0 ? row[c] : 0.f;
    const float b = in1 ? row[c + 1] : 0.f;
    s0 += a;
    s1 += b;
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    *reinterpret_cast<bf16x2_t*>(dzp + r * Cp + c) = bf16x2_t{(bf16)a, (bf16)b};
  }
  if (part) {
    if (in0) part[(int64_t)blockIdx.y * C + c] = s0;
    if (in1) part[(int64_t)blockIdx.y * C + c + 1] = s1;
  }
}

// db[c] = sum over the partial rows: a workgroup per 64 columns, wave w of kColsumWaves summing
// partial rows [w nq, (w + 1) nq) with eight loads in flight (eight running sums, added in
// order), the waves' sums added in wave order through LDS: a fixed order, so the result is
// deterministic.
constexpr int kColsumWaves = 16;

__global__ __launch_bounds__(64 * kColsumWaves) void logit_grad_colsum_kernel(const float* __restrict__ part,
                                                                              int nblk, int64_t C,
                                                                              float* __restrict__ db) {
  __shared__ float red[kColsumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int nq = (nblk + kColsumWaves - 1) / kColsumWaves;
  const int i0 = wave * nq, i1 = min(nblk, i0 + nq);
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.f;
  if (c < C) {
    for (int i = i0; i < i1; i += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (i + u < i1) acc[u] += part[(int64_t)(i + u) * C + c];
    }
  }
  float s = acc[0];
#pragma unroll
  for (int u = 1; u < 8; ++u) s += acc[u];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < C) {
    float t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kColsumWaves; ++w) t += red[w][lane];
    db[c] = t;
  }
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
  MOC_REQUIRE(C <= kMaxRouterC, MOC_ERR_UNSUPPORTED, "moc_router_topk: C=%lld exceeds %d", (long long)C, kMaxRouterC);
  if (R == 0) return MOC_OK;
  if (router_wave_rows(R, C, k)) {
    if (C <= 64 * kWaveShortE)
      hipLaunchKernelGGL(router_topk_wave_kernel<kWaveShortE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, R, C, S, k, idx, w, probs, 0.f, nullptr, nullptr);
    else
      hipLaunchKernelGGL(router_topk_wave_kernel<kWaveMaxE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, R, C, S, k, idx, w, probs, 0.f, nullptr, nullptr);
    return check_launch("router_topk_wave_kernel");
  }
  const size_t lds = (size_t)C * sizeof(float);
  if (router_threads(R) == 1024)
    hipLaunchKernelGGL(router_topk_kernel<1024>, dim3((unsigned)R), dim3(1024), lds, stream, logits, C, S, k, idx, w,
                       probs, 0.f, nullptr, nullptr);
  else
    hipLaunchKernelGGL(router_topk_kernel<256>, dim3((unsigned)R), dim3(256), lds, stream, logits, C, S, k, idx, w,
                       probs, 0.f, nullptr, nullptr);
  return check_launch("router_topk_kernel");
}

int moc_router_topk_prepend(const float* logits, int64_t R, int64_t C, int S, int k, float scale, int32_t* idx,
                            float* w, int32_t* idx_star, float* omega, hipStream_t stream) {
  MOC_REQUIRE(logits && idx && w && idx_star && omega, MOC_ERR_ARG, "moc_router_topk_prepend: null pointer");
  MOC_REQUIRE(R >= 0 && C > 0, MOC_ERR_ARG, "moc_router_topk_prepend: bad shape R=%lld C=%lld", (long long)R,
              (long long)C);
  MOC_REQUIRE(S > 0 && S <= C, MOC_ERR_ARG, "moc_router_topk_prepend: needs 0 < S <= C, got S=%d", S);
  MOC_REQUIRE(k > 0 && k <= C - S, MOC_ERR_ARG, "moc_router_topk_prepend: k=%d must be in [1, C-S=%lld]", k,
              (long long)(C - S));
  MOC_REQUIRE(k <= kMaxTopK, MOC_ERR_UNSUPPORTED, "moc_router_topk_prepend: k=%d exceeds %d", k, kMaxTopK);
  MOC_REQUIRE(C <= kMaxRouterC, MOC_ERR_UNSUPPORTED, "moc_router_topk_prepend: C=%lld exceeds %d", (long long)C,
              kMaxRouterC);
  if (R == 0) return MOC_OK;
  if (router_wave_rows(R, C, k)) {
    if (C <= 64 * kWaveShortE)
      hipLaunchKernelGGL(router_topk_wave_kernel<kWaveShortE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, R, C, S, k, idx, w, nullptr, scale, idx_star, omega);
    else
      hipLaunchKernelGGL(router_topk_wave_kernel<kWaveMaxE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, R, C, S, k, idx, w, nullptr, scale, idx_star, omega);
    return check_launch("router_topk_wave_kernel(prepend)");
  }
  const size_t lds = (size_t)C * sizeof(float);
  if (router_threads(R) == 1024)
    hipLaunchKernelGGL(router_topk_kernel<1024>, dim3((unsigned)R), dim3(1024), lds, stream, logits, C, S, k, idx, w,
                       nullptr, scale, idx_star, omega);
  else
    hipLaunchKernelGGL(router_topk_kernel<256>, dim3((unsigned)R), dim3(256), lds, stream, logits, C, S, k, idx, w,
                       nullptr, scale, idx_star, omega);
  return check_launch("router_topk_kernel(prepend)");
}

int moc_router_topk_bwd(const float* logits, const int32_t* idx, const float* dw, int64_t R, int64_t C, int S, int k,
                        float* dlogits, hipStream_t stream) {
  MOC_REQUIRE(logits && idx && dw && dlogits, MOC_ERR_ARG, "moc_router_topk_bwd: null pointer");
  MOC_REQUIRE(S >= 0 && S <= C && k > 0 && k <= C - S && k <= kMaxTopK, MOC_ERR_ARG,
              "moc_router_topk_bwd: bad S=%d k=%d C=%lld", S, k, (long long)C);
  MOC_REQUIRE(C <= kMaxRouterC / 2, MOC_ERR_UNSUPPORTED, "moc_router_topk_bwd: C=%lld exceeds %d", (long long)C,
              kMaxRouterC / 2);
  if (R == 0) return MOC_OK;
  if (router_wave_rows(R, C, k)) {
    if (C <= 64 * kWaveShortE)
      hipLaunchKernelGGL(router_topk_bwd_wave_kernel<kWaveShortE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, idx, dw, R, C, S, k, nullptr, dlogits);
    else
      hipLaunchKernelGGL(router_topk_bwd_wave_kernel<kWaveMaxE>, dim3((unsigned)((R + kWaveRows - 1) / kWaveRows)),
                         dim3(64 * kWaveRows), 0, stream, logits, idx, dw, R, C, S, k, nullptr, dlogits);
    return check_launch("router_topk_bwd_wave_kernel");
  }
  const size_t lds = 2 * (size_t)C * sizeof(float);
  if (router_threads(R) == 1024)
    hipLaunchKernelGGL(router_topk_bwd_kernel<1024>, dim3((unsigned)R), dim3(1024), lds, stream, logits, idx, dw, C, S,
                       k, dlogits);
  else
    hipLaunchKernelGGL(router_topk_bwd_kernel<256>, dim3((unsigned)R), dim3(256), lds, stream, logits, idx, dw, C, S, k,
                       dlogits);
  return check_launch("router_topk_bwd_kernel");
}

int moc_router_seq_bwd(const float* logits, const int32_t* idx, const float* w, const float* dom_part, int HK,
                       int64_t R, int64_t C, int S, int k, float scale, const float* dz_in, float* dlogits,
                       hipStream_t stream) {
  MOC_REQUIRE(logits && idx && w && dom_part && dlogits, MOC_ERR_ARG, "moc_router_seq_bwd: null pointer");
  MOC_REQUIRE(HK > 0 && S > 0 && S <= C && k > 0 && k <= C - S, MOC_ERR_ARG,
              "moc_router_seq_bwd: bad HK=%d S=%d k=%d C=%lld", HK, S, k, (long long)C);
  MOC_REQUIRE(k <= kMaxTopK && S <= kMaxSeqShared && C <= kMaxRouterC / 2, MOC_ERR_UNSUPPORTED,
              "moc_router_seq_bwd: k=%d, S=%d or C=%lld beyond %d / %d / %d", k, S, (long long)C, kMaxTopK,
              kMaxSeqShared, kMaxRouterC / 2);
  if (R == 0) return MOC_OK;
  const size_t lds = 2 * (size_t)C * sizeof(float);
  if (router_threads(R) == 1024)
    hipLaunchKernelGGL(router_seq_bwd_kernel<1024>, dim3((unsigned)R), dim3(1024), lds, stream, logits, idx, w,
                       dom_part, HK, C, S, k, scale, dz_in, dlogits);
  else
    hipLaunchKernelGGL(router_seq_bwd_kernel<256>, dim3((unsigned)R), dim3(256), lds, stream, logits, idx, w, dom_part,
                       HK, C, S, k, scale, dz_in, dlogits);
  return check_launch("router_seq_bwd_kernel");
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

namespace {
int pool_splits(int64_t B, int64_t L) {
  // ~16 rows per workgroup, at most 256 splits, at least ~512 workgroups when L allows
  int64_t n = (L + 15) / 16;
  if (n > 256) n = 256;
  return (int)(n < 1 ? 1 : n);
}
}  // namespace

size_t moc_router_pool_workspace(int64_t B, int64_t L, int64_t d) {
  return (size_t)pool_splits(B, L) * B * d * sizeof(float);
}

int moc_router_pool(const void* h, int dtype, int64_t B, int64_t L, int64_t d, const float* coef, float* pooled,
                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  MOC_REQUIRE(h && pooled && workspace, MOC_ERR_ARG, "moc_router_pool: null pointer");
  MOC_REQUIRE(B >= 0 && L > 0 && d > 0, MOC_ERR_ARG, "moc_router_pool: bad shape");
  MOC_REQUIRE(workspace_bytes >= moc_router_pool_workspace(B, L, d), MOC_ERR_ARG, "moc_router_pool: workspace too small");
  MOC_REQUIRE(B < 65536, MOC_ERR_UNSUPPORTED, "moc_router_pool: B=%lld too large", (long long)B);
  if (B == 0) return MOC_OK;
  const int nsplit = pool_splits(B, L);
  const int rows = (int)((L + nsplit - 1) / nsplit);
  dim3 grid((unsigned)B, (unsigned)nsplit);
  float* part = (float*)workspace;
  const bool vec = d % 8 == 0 && ((uintptr_t)h & 31) == 0;
  if (!vec) {
    if (dtype == MOC_F32)
      hipLaunchKernelGGL(pool_partial_cols_kernel<float>, grid, dim3(kPoolThreads), 0, stream, (const float*)h, L, d,
                         coef, rows, part);
    else if (dtype == MOC_BF16)
      hipLaunchKernelGGL(pool_partial_cols_kernel<bf16>, grid, dim3(kPoolThreads), 0, stream, (const bf16*)h, L, d,
                         coef, rows, part);
    else
      return set_error(MOC_ERR_UNSUPPORTED, "moc_router_pool: dtype %d", dtype);
  } else if (dtype == MOC_F32)
    hipLaunchKernelGGL(pool_partial_kernel<float>, grid, dim3(kPoolThreads), 0, stream, (const float*)h, L, d, coef,
                       rows, part);
  else if (dtype == MOC_BF16)
    hipLaunchKernelGGL(pool_partial_kernel<bf16>, grid, dim3(kPoolThreads), 0, stream, (const bf16*)h, L, d, coef,
                       rows, part);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_pool: dtype %d", dtype);
  int rc = check_launch("pool_partial_kernel");
  if (rc) return rc;
  const float inv = coef ? 1.f : 1.f / (float)L;
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((B * d + 63) / 64)), dim3(256), 0, stream, part, nsplit, B, d,
                     inv, pooled);
  return check_launch("pool_reduce_kernel");
}

int moc_router_pool1(const void* h, int dtype, int64_t B, int64_t L, int64_t d, const float* coef, float* pooled,
                     hipStream_t stream) {
  MOC_REQUIRE(h && pooled, MOC_ERR_ARG, "moc_router_pool1: null pointer");
  MOC_REQUIRE(B >= 0 && L > 0 && d > 0 && B < 65536, MOC_ERR_ARG, "moc_router_pool1: bad shape");
  MOC_REQUIRE(d % 8 == 0 && ((uintptr_t)h & 15) == 0, MOC_ERR_UNSUPPORTED,
              "moc_router_pool1: d=%lld must be a multiple of 8 with 16-byte aligned rows", (long long)d);
  if (B == 0) return MOC_OK;
  const dim3 grid((unsigned)((d + 63) / 64), (unsigned)B);
  const float scale = coef ? 1.f : 1.f / (float)L;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(pool_single_kernel<bf16>, grid, dim3(1024), 0, stream, (const bf16*)h, L, d, coef, scale,
                       pooled);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(pool_single_kernel<float>, grid, dim3(1024), 0, stream, (const float*)h, L, d, coef, scale,
                       pooled);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_pool1: dtype %d", dtype);
  return check_launch("pool_single_kernel");
}

int moc_rows_add_bcast(void* x, int dtype, int64_t B, int64_t L, int64_t d, const float* v, const float* coef,
                       float scale, hipStream_t stream) {
  MOC_REQUIRE(x && v, MOC_ERR_ARG, "moc_rows_add_bcast: null pointer");
  MOC_REQUIRE(B >= 0 && L >= 0 && d > 0 && d % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)v & 15) == 0,
              MOC_ERR_UNSUPPORTED, "moc_rows_add_bcast: d=%lld must be a multiple of 8, pointers 16-byte aligned",
              (long long)d);
  const int64_t n = B * L * (d / 8);
  if (n == 0) return MOC_OK;
  MOC_REQUIRE(n < ((int64_t)1 << 39), MOC_ERR_UNSUPPORTED, "moc_rows_add_bcast: too large");
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(rows_add_bcast_kernel<bf16>, grid, dim3(256), 0, stream, (bf16*)x, B, L, d, v, coef, scale);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(rows_add_bcast_kernel<float>, grid, dim3(256), 0, stream, (float*)x, B, L, d, v, coef, scale);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_rows_add_bcast: dtype %d", dtype);
  return check_launch("rows_add_bcast_kernel");
}

int moc_router_linear(const float* x, int64_t R, int64_t d, const void* W, int w_dtype, const float* bias, int64_t C,
                      float* logits, hipStream_t stream) {
  MOC_REQUIRE(x && W && logits, MOC_ERR_ARG, "moc_router_linear: null pointer");
  MOC_REQUIRE(R >= 0 && d > 0 && C > 0, MOC_ERR_ARG, "moc_router_linear: bad shape");
  MOC_REQUIRE(d <= 4096 && d % 4 == 0, MOC_ERR_UNSUPPORTED, "moc_router_linear: d=%lld must be a multiple of 4, <= 4096",
              (long long)d);
  if (R == 0) return MOC_OK;
  if (d % 64 == 0 && d <= 64 * 16 * 4) {
    // matrix-core version: W chunks for d <= 1,024 fully in registers (12 blocks at d = 768)
    const dim3 g16((unsigned)((C + 15) / 16));
    if (w_dtype == MOC_F32)
      hipLaunchKernelGGL((router_linear_mfma_kernel<float, 16>), g16, dim3(256), 0, stream, x, R, d, (const float*)W,
                         bias, C, logits);
    else if (w_dtype == MOC_BF16)
      hipLaunchKernelGGL((router_linear_mfma_kernel<bf16, 16>), g16, dim3(256), 0, stream, x, R, d, (const bf16*)W,
                         bias, C, logits);
    else
      return set_error(MOC_ERR_UNSUPPORTED, "moc_router_linear: dtype %d", w_dtype);
    return check_launch("router_linear_mfma_kernel");
  }
  dim3 grid((unsigned)((C + kLinChapFwd - 1) / kLinChapFwd));
  // only the rows of one chunk: small batches leave room for more resident workgroups
  const size_t lds = (size_t)std::min<int64_t>(R, kLinRows) * d * sizeof(float);
  if (w_dtype == MOC_F32)
    hipLaunchKernelGGL(router_linear_kernel<float>, grid, dim3(256), lds, stream, x, R, d, (const float*)W, bias, C,
                       logits);
  else if (w_dtype == MOC_BF16)
    hipLaunchKernelGGL(router_linear_kernel<bf16>, grid, dim3(256), lds, stream, x, R, d, (const bf16*)W, bias, C,
                       logits);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_linear: dtype %d", w_dtype);
  return check_launch("router_linear_kernel");
}

size_t moc_router_linear_bwd_workspace(int64_t R, int64_t d, int64_t C) {
  return (size_t)((C + kLinChap - 1) / kLinChap) * R * d * sizeof(float);
}

int moc_router_linear_bwd(const float* dz, const float* x, int64_t R, int64_t d, const void* W, int w_dtype, int64_t C,
                          float* dx, float* dW, float* db, void* workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  MOC_REQUIRE(dz && x && W, MOC_ERR_ARG, "moc_router_linear_bwd: null pointer");
  MOC_REQUIRE(d <= 4096 && d % 4 == 0, MOC_ERR_UNSUPPORTED,
              "moc_router_linear_bwd: d=%lld must be a multiple of 4, <= 4096", (long long)d);
  if (R == 0 || (!dx && !dW && !db)) return MOC_OK;
  const int64_t nwg = (C + kLinChap - 1) / kLinChap;
  float* part = nullptr;
  if (dx) {
    MOC_REQUIRE(workspace && workspace_bytes >= moc_router_linear_bwd_workspace(R, d, C), MOC_ERR_ARG,
                "moc_router_linear_bwd: workspace too small");
    part = (float*)workspace;
  }
  const size_t lds = (size_t)kLinRows * d * sizeof(float);
  if (w_dtype == MOC_F32)
    hipLaunchKernelGGL(router_linear_bwd_kernel<float>, dim3((unsigned)nwg), dim3(256), lds, stream, dz, x, R, d,
                       (const float*)W, C, dW, db, part);
  else if (w_dtype == MOC_BF16)
    hipLaunchKernelGGL(router_linear_bwd_kernel<bf16>, dim3((unsigned)nwg), dim3(256), lds, stream, dz, x, R, d,
                       (const bf16*)W, C, dW, db, part);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_router_linear_bwd: dtype %d", w_dtype);
  int rc = check_launch("router_linear_bwd_kernel");
  if (rc || !dx) return rc;
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((R * d + 63) / 64)), dim3(256), 0, stream, part, (int)nwg, R,
                     d, 1.f, dx);
  return check_launch("pool_reduce_kernel");
}

size_t moc_router_losses_workspace(int64_t R, int64_t C) {
  const int64_t nsplit = (R + kLossColRows - 1) / kLossColRows;
  // column-sum partials [nsplit][2][C], column sums [2][C], row entropies [R]
  return (size_t)(nsplit * 2 * C + 2 * C + R) * sizeof(float);
}

int moc_router_losses(const float* logits, int64_t R, int64_t C, const int32_t* idx, int k, float* row_lse,
                      float* col_coef, int32_t* counts, float* losses, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  MOC_REQUIRE(logits && row_lse && col_coef && counts && losses && workspace && (idx || k == 0), MOC_ERR_ARG,
              "moc_router_losses: null pointer");
  MOC_REQUIRE(R > 0 && C > 0 && k >= 0, MOC_ERR_ARG, "moc_router_losses: bad shape R=%lld C=%lld k=%d", (long long)R,
              (long long)C, k);
  MOC_REQUIRE(C <= kMaxRouterC, MOC_ERR_UNSUPPORTED, "moc_router_losses: C=%lld exceeds %d", (long long)C, kMaxRouterC);
  MOC_REQUIRE(R < ((int64_t)1 << 31) / 4, MOC_ERR_UNSUPPORTED, "moc_router_losses: too many rows");
  MOC_REQUIRE(workspace_bytes >= moc_router_losses_workspace(R, C), MOC_ERR_ARG, "moc_router_losses: workspace too small");
  MOC_REQUIRE(((uintptr_t)col_coef & 7) == 0 && ((uintptr_t)workspace & 3) == 0, MOC_ERR_ARG,
              "moc_router_losses: col_coef must be 8-byte and workspace 4-byte aligned");
  const int64_t nsplit = (R + kLossColRows - 1) / kLossColRows;
  float* part = (float*)workspace;
  float* col_sums = part + nsplit * 2 * C;
  float* row_ent = col_sums + 2 * C;
  const unsigned cblk = (unsigned)((C + kLossThreads - 1) / kLossThreads);
  hipLaunchKernelGGL(router_loss_zero_kernel, dim3(cblk), dim3(kLossThreads), 0, stream, counts, C);
  int rc = check_launch("router_loss_zero_kernel");
  if (rc) return rc;
  if (C <= kLossThreads * kLossRowCols)
    hipLaunchKernelGGL(router_loss_rowstats_block_kernel, dim3((unsigned)R), dim3(kLossThreads), 0, stream, logits, R,
                       C, idx, k, row_lse, row_ent, counts);
  else
    hipLaunchKernelGGL(router_loss_rowstats_kernel, dim3((unsigned)((R + 3) / 4)), dim3(kLossThreads), 0, stream,
                       logits, R, C, idx, k, row_lse, row_ent, counts);
  rc = check_launch("router_loss_rowstats_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(router_loss_colsum_kernel, dim3(cblk, (unsigned)nsplit), dim3(kLossThreads), 0, stream, logits,
                     R, C, row_lse, part);
  rc = check_launch("router_loss_colsum_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)((2 * C + 63) / 64)), dim3(256), 0, stream, part, (int)nsplit,
                     (int64_t)1, 2 * C, 1.f, col_sums);
  rc = check_launch("pool_reduce_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(router_loss_final_kernel, dim3(1), dim3(kLossFinalThreads), 0, stream, col_sums, row_lse, row_ent,
                     counts, R, C, losses, (float2*)col_coef);
  return check_launch("router_loss_final_kernel");
}

int moc_router_losses_bwd(const float* logits, int64_t R, int64_t C, const float* row_lse, const float* col_coef,
                          const float* dlosses, float* dlogits, hipStream_t stream) {
  MOC_REQUIRE(logits && row_lse && col_coef && dlosses && dlogits, MOC_ERR_ARG, "moc_router_losses_bwd: null pointer");
  MOC_REQUIRE(R > 0 && C > 0 && R < ((int64_t)1 << 31), MOC_ERR_ARG, "moc_router_losses_bwd: bad shape");
  MOC_REQUIRE(((uintptr_t)col_coef & 7) == 0, MOC_ERR_ARG, "moc_router_losses_bwd: col_coef must be 8-byte aligned");
  const float2* cf = (const float2*)col_coef;
  if (C <= kLossThreads * kLossRowCols)
    hipLaunchKernelGGL(router_loss_bwd_block_kernel, dim3((unsigned)R), dim3(kLossThreads), 0, stream, logits, R, C,
                       row_lse, cf, dlosses, dlogits);
  else
    hipLaunchKernelGGL(router_loss_bwd_kernel, dim3((unsigned)((R + 3) / 4)), dim3(kLossThreads), 0, stream, logits,
                       R, C, row_lse, cf, dlosses, dlogits);
  return check_launch("router_loss_bwd_kernel");
}


size_t moc_router_topk_bwd_pack_workspace(int64_t R, int64_t C) {
  if (R <= 0 || C <= 0) return 0;
  const int64_t per = (int64_t)kWaveRows * kPackWaveRows;
  return (size_t)((R + per - 1) / per) * (size_t)C * sizeof(float);
}

int moc_router_topk_bwd_pack(const float* logits, const int32_t* idx, const float* dw, int64_t R, int64_t C, int S,
                             int k, const float* dz_in, int64_t Cp, void* dzp, float* db, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  MOC_REQUIRE(logits && idx && dw && dzp && db && workspace, MOC_ERR_ARG, "moc_router_topk_bwd_pack: null pointer");
  MOC_REQUIRE(S >= 0 && S <= C && k > 0 && k <= C - S, MOC_ERR_ARG, "moc_router_topk_bwd_pack: bad S=%d k=%d C=%lld",
              S, k, (long long)C);
  MOC_REQUIRE(R > 64 && C <= 64 * kWaveMaxE && k <= kWaveMaxK, MOC_ERR_UNSUPPORTED,
              "moc_router_topk_bwd_pack: needs R > 64, C <= %d, k <= %d (R=%lld C=%lld k=%d)", 64 * kWaveMaxE,
              kWaveMaxK, (long long)R, (long long)C, k);
  MOC_REQUIRE(Cp >= C && Cp <= 64 * kWaveMaxE && Cp % 2 == 0 && R * Cp < ((int64_t)1 << 40), MOC_ERR_ARG,
              "moc_router_topk_bwd_pack: Cp=%lld (>= C, even, <= %d)", (long long)Cp, 64 * kWaveMaxE);
  MOC_REQUIRE(((uintptr_t)dzp & 3) == 0, MOC_ERR_ARG, "moc_router_topk_bwd_pack: dzp must be 4-byte aligned");
  MOC_REQUIRE(workspace_bytes >= moc_router_topk_bwd_pack_workspace(R, C), MOC_ERR_ARG,
              "moc_router_topk_bwd_pack: workspace too small");
  const int64_t per = (int64_t)kWaveRows * kPackWaveRows;
  const int nblk = (int)((R + per - 1) / per);
  if (dz_in)
    hipLaunchKernelGGL((router_topk_bwd_pack_kernel<true, kWaveMaxE>), dim3((unsigned)nblk), dim3(64 * kWaveRows), 0, stream,
                       logits, idx, dw, R, C, S, k, dz_in, Cp, (bf16*)dzp, (float*)workspace);
  else
    hipLaunchKernelGGL((router_topk_bwd_pack_kernel<false, kWaveMaxE>), dim3((unsigned)nblk), dim3(64 * kWaveRows), 0, stream,
                       logits, idx, dw, R, C, S, k, dz_in, Cp, (bf16*)dzp, (float*)workspace);
  if (int rc = check_launch("router_topk_bwd_pack_kernel")) return rc;
  hipLaunchKernelGGL(logit_grad_colsum_kernel, dim3((unsigned)((C + 63) / 64)), dim3(64 * kColsumWaves), 0, stream,
                     (const float*)workspace, nblk, C, db);
  return check_launch("logit_grad_colsum_kernel");
}

size_t moc_logit_grad_pack_workspace(int64_t R, int64_t C) {
  if (R <= 0 || C <= 0) return 0;
  return (size_t)((R + kPackRows - 1) / kPackRows) * (size_t)C * sizeof(float);
}

int moc_logit_grad_pack(const float* dz, int64_t R, int64_t C, int64_t Cp, void* dzp, float* db, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  MOC_REQUIRE(dz && dzp, MOC_ERR_ARG, "moc_logit_grad_pack: null pointer");
  MOC_REQUIRE(R > 0 && C > 0 && Cp >= C && Cp % 2 == 0 && R * Cp < ((int64_t)1 << 40), MOC_ERR_ARG,
              "moc_logit_grad_pack: R=%lld C=%lld Cp=%lld (Cp >= C, even)", (long long)R, (long long)C,
              (long long)Cp);
  MOC_REQUIRE(((uintptr_t)dzp & 3) == 0, MOC_ERR_ARG, "moc_logit_grad_pack: dzp must be 4-byte aligned");
  MOC_REQUIRE(!db || (workspace && workspace_bytes >= moc_logit_grad_pack_workspace(R, C)), MOC_ERR_ARG,
              "moc_logit_grad_pack: workspace too small");
  const int nblk = (int)((R + kPackRows - 1) / kPackRows);
  MOC_REQUIRE(nblk < 65536, MOC_ERR_UNSUPPORTED, "moc_logit_grad_pack: R=%lld too large", (long long)R);
  const dim3 grid((unsigned)((Cp / 2 + 255) / 256), (unsigned)nblk);
  hipLaunchKernelGGL(logit_grad_pack_kernel, grid, dim3(256), 0, stream, dz, R, C, Cp, (bf16*)dzp,
                     db ? (float*)workspace : nullptr);
  if (int rc = check_launch("logit_grad_pack_kernel")) return rc;
  if (!db) return MOC_OK;
  hipLaunchKernelGGL(logit_grad_colsum_kernel, dim3((unsigned)((C + 63) / 64)), dim3(64 * kColsumWaves), 0, stream,
                     (const float*)workspace, nblk, C, db);
  return check_launch("logit_grad_colsum_kernel");
}

}  // extern "C"
