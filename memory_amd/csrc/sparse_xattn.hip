// Token-routed sparse memory attention (every query token picks its own
// chapters), forward and backward, chapter-centric.
//
// Inputs: q [tokens][HQ][64] (token = b * Tq + t), K / V addressed by element
// strides (chapter cs, kv-head hs, row rs) so both the per-batch natural layout
// [B*Tk][HK][64] of the reference's FSA entry points and the chapter-head tiles
// of kv_project work.  An edge e = token * S + slot selects chapter gid; the
// chapter plan (plan.hip) groups edges per distinct chapter.  Rows of an edge
// are the query heads hq it serves: rpe rows per edge, row r <-> hq = hq_off + r.
//
// Forward = two kernels:
//   sparse_fwd_kernel      per (chapter, kv head): for every row of every edge of
//                          the chapter, the softmax over the chapter's 64 keys is
//                          complete inside the tile -> o_part (normalised) and
//                          lse_part (log2 domain).
//   sparse_combine_kernel  per (token, head) over its S slots:
//     mode 0 (MoE, kernels-final/kernel_v4.py:1-15 / naive_reference_weighted,
//             benchmark_kernels_final.py:239-294):  o = sum_s w_s o_s
//     mode 1 (joint, kernel_v2.py / naive_reference_unweighted :206-236):
//             o = sum_s a_s o_s / sum_s a_s,  a_s = exp2(lse_s)
//     mode 2 (block weights, kernel_v2.py:765-773): a_s = max(w_s, 0) exp2(lse_s)
//     mode 3 (joint log-bias, kernel_v5.py:1-9, :218-220): a_s = max(w_s, 1e-20) exp2(lse_s)
//     and the joint log-sum-exp of the row for the backward (modes 1-3).
// Backward: prep (per-slot dw for mode 0, row delta for modes 1-3), the
// chapter-centric kernel (dK / dV accumulated in registers over all edges of the
// chapter -- deterministic, no atomics --, per-edge dQ parts, per-edge
// d log(weight) for modes 2-3), then per-token reductions of dQ and dw.
#include "moc_common.h"

namespace moc {

constexpr int kSpDh = 64;

template <typename T> struct SpCfg;
template <> struct SpCfg<bf16> { static constexpr int NW = 4; };
template <> struct SpCfg<float> { static constexpr int NW = 2; };
template <typename T> constexpr int sp_threads() { return 64 * SpCfg<T>::NW; }

// Load a 64x64 K or V tile at (chapter gid, head hk) into LDS as [key][dim]
// (transpose = false) or [dim][key] (transpose = true).
template <typename T, int NT>
__device__ __forceinline__ void sp_load_tile(char* dst, const T* base, int64_t rs, int tid, bool transpose) {
  using Tile = SwzTile<T, 64>;
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int CPR = 64 / EPC;
  for (int i = tid; i < 64 * CPR; i += NT) {
    const int row = i / CPR, c0 = (i % CPR) * EPC;
    V16 v = ld16(base + row * rs + c0);
    if (!transpose) {
      st16(dst + Tile::off(row, c0), v);
    } else {
      const T* t = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int x = 0; x < EPC; ++x) *reinterpret_cast<T*>(dst + Tile::off(c0 + x, row)) = t[x];
    }
  }
}

// ------------------------------------------------------------------ forward
// Partial rows (per (edge, row) outputs and dQ contributions) are kept in the data type of the
// call: bf16 for bf16 inputs (half the bytes of the round trip through HBM), f32 for f32.
__device__ __forceinline__ f32x4 part_load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 part_load4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ void part_store4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void part_store4(bf16* p, f32x4 v) {
  bf16x4 o;
#pragma unroll
  for (int x = 0; x < 4; ++x) o[x] = (bf16)v[x];
  *reinterpret_cast<bf16x4*>(p) = o;
}

template <typename T>
__global__ __launch_bounds__(64 * SpCfg<T>::NW) void sparse_fwd_kernel(
    const T* __restrict__ q, int HQ, const T* __restrict__ k, const T* __restrict__ v, int64_t cs, int64_t hs,
    int64_t rs, int HK, const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq,
    const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge, int S, int hk0, int hq_off, int rpe,
    float scale_log2, T* __restrict__ o_part, float* __restrict__ lse_part, const float* __restrict__ omega) {
  typedef typename Frag<T>::type F8;
  constexpr int NW = SpCfg<T>::NW, NT = 64 * NW;
  using Tile = SwzTile<T, 64>;
  constexpr int TB = 64 * 64 * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) char sK[TB];
  __shared__ __attribute__((aligned(16))) char sVt[TB];
  const int u = blockIdx.x, hk = hk0 + blockIdx.y;
  if (u >= n_uniq[0]) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int gid = uniq[u];
  sp_load_tile<T, NT>(sK, k + gid * cs + hk * hs, rs, tid, false);
  sp_load_tile<T, NT>(sVt, v + gid * cs + hk * hs, rs, tid, true);
  __syncthreads();
  const int G = HQ / HK;
  const int p0 = csr_off[u], p1 = csr_off[u + 1];
  const int nrows = (p1 - p0) * G;
  for (int r0 = 32 * wave; r0 < nrows; r0 += 32 * NW) {
    F8 qf[2][2];
    int erow[2];  // e * rpe + row, or -1
    float wrow[2] = {1.f, 1.f};
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int r = r0 + 16 * qb + c16;
      erow[qb] = -1;
      if (r < nrows) {
        const int e = csr_edge[p0 + r / G];
        const int hq = hk * G + r % G;
        const int64_t tok = e / S;
        erow[qb] = e * rpe + (hq - hq_off);
        if (omega) wrow[qb] = omega[e];
        const T* qp = q + ((size_t)tok * HQ + hq) * kSpDh;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) qf[qb][ks] = Load8<T, T>::run(qp + 32 * ks + 8 * g);
      } else {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) qf[qb][ks] = zero_frag<T>();
      }
    }
    f32x4 st[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        F8 a = Tile::frag(sK, 16 * kb + c16, 32 * ks + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) mma(st[kb][qb], a, qf[qb][ks]);
      }
    F8 pf[2][2];
    float m[2], l[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int x = 0; x < 4; ++x) mx = fmaxf(mx, st[kb][qb][x]);
      const float c = wrow[qb] * scale_log2;
      m[qb] = quad_max(mx) * c;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const float p = exp2f(st[kb][qb][x] * c - m[qb]);
          ps += p;
          st[kb][qb][x] = p;
        }
      l[qb] = quad_sum(ps);
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          pf[qb][ks2][x] = from_f<T>(st[2 * ks2][qb][x]);
          pf[qb][ks2][4 + x] = from_f<T>(st[2 * ks2 + 1][qb][x]);
        }
    }
    f32x4 o[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        F8 a = Tile::frag44(sVt, 16 * db + c16, 32 * ks2 + 4 * g, 32 * ks2 + 16 + 4 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) mma(o[db][qb], a, pf[qb][ks2]);
      }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if (erow[qb] < 0) continue;
      const float inv = wrow[qb] / l[qb];
      T* op = o_part + (size_t)erow[qb] * kSpDh;
#pragma unroll
      for (int db = 0; db < 4; ++db) part_store4(op + 16 * db + 4 * g, o[db][qb] * inv);
      if (g == 0) lse_part[erow[qb]] = m[qb] + log2f(l[qb]);
    }
  }
}

// Per (token, row): combine the slot partials.  One wave per row: the slot weights a_s live one
// per lane (64-slot chunks); the partial rows are read as 16-byte pieces, a row of 64 dims being
// LPR lanes (8 for bf16, 16 for f32) and lane group sg = lane / LPR streaming the rows of slots
// sg, sg + NG, ... (four loads in flight per lane); the NG groups are added in a fixed order.
// (Right after the kernels that wrote them, 16-byte loads of these rows take about half the time
// of 8-byte ones.)
__device__ __forceinline__ float sp_logw(int mode, float w) {
  if (mode == 2) return w > 0.f ? log2f(w) : -INFINITY;
  if (mode == 3) return log2f(fmaxf(w, 1e-20f));
  return 0.f;
}

template <typename P> struct SpRow16 {
  static constexpr int EPL = 16 / (int)sizeof(P);   // elements per lane and load
  static constexpr int LPR = 64 / EPL;              // lanes per 64-dim row
  static constexpr int NG = 64 / LPR;               // rows per load instruction
  typedef typename std::conditional<sizeof(P) == 2, bf16x8, f32x4>::type V;
};

// acc += sum over the slots s0 .. s0 + 63 of one row of a_s * part row (lane s - s0 holds a_s);
// a_s = 0 marks a skipped slot, whose partial row is never read.
template <typename P>
__device__ __forceinline__ void sp_slot_sum(const P* __restrict__ part, int64_t tok, int S, int rpe, int r, float a,
                                            int s0, int lane, float (&acc)[SpRow16<P>::EPL]) {
  using R = SpRow16<P>;
  const int sg = lane / R::LPR, ch = lane % R::LPR;
  const int n = min(64, S - s0);
  const int iters = (n + R::NG - 1) / R::NG;   // wave-uniform trip count
  for (int k0 = 0; k0 < iters; k0 += 4) {
    typename R::V v[4];
    float av[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = R::NG * (k0 + i) + sg;
      const float aj = __shfl(a, j & 63, 64);
      av[i] = j < n ? aj : 0.f;
      v[i] = typename R::V{};
      if (av[i] != 0.f) {
        const int64_t e = tok * S + s0 + j;
        v[i] = *reinterpret_cast<const typename R::V*>(part + (e * rpe + r) * kSpDh + R::EPL * ch);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int x = 0; x < R::EPL; ++x) acc[x] += av[i] * (float)v[i][x];
  }
}

// sum over the NG lane groups (lane bits LPR .. 32), in a fixed order
template <typename P>
__device__ __forceinline__ void sp_groups_sum(float (&acc)[SpRow16<P>::EPL]) {
  using R = SpRow16<P>;
#pragma unroll
  for (int o = R::LPR; o < 64; o <<= 1)
#pragma unroll
    for (int x = 0; x < R::EPL; ++x) acc[x] += __shfl_xor(acc[x], o, 64);
}

// lanes < LPR store the row's 64 values (16 bytes each)
template <typename T>
__device__ __forceinline__ void sp_row_store(T* __restrict__ row, const float (&acc)[SpRow16<T>::EPL], float scale,
                                             int lane) {
  using R = SpRow16<T>;
  if (lane < R::LPR) {
    typename R::V o;
#pragma unroll
    for (int x = 0; x < R::EPL; ++x) o[x] = from_f<T>(acc[x] * scale);
    *reinterpret_cast<typename R::V*>(row + R::EPL * lane) = o;
  }
}

constexpr int kCombWaves = 4;

template <typename T>
__global__ __launch_bounds__(64 * kCombWaves) void sparse_combine_kernel(const T* __restrict__ o_part,
                                                                         const float* __restrict__ lse_part,
                                                                         const int32_t* __restrict__ edge_u,
                                                                         const float* __restrict__ w, int mode, int S,
                                                                         int rpe, int64_t ntok, int HQ, int hq_off,
                                                                         T* __restrict__ out,
                                                                         float* __restrict__ lse_joint) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kCombWaves + (threadIdx.x >> 6);
  if (row >= ntok * rpe) return;
  const int64_t tok = row / rpe;
  const int r = (int)(row % rpe);
  // slot weights: mode 0 a_s = w_s; joint modes a_s = 2^(lse_s + log w_s - M)
  float M = -INFINITY;
  if (mode != 0) {
    for (int s0 = 0; s0 < S; s0 += 64) {
      const int s = s0 + lane;
      if (s < S) {
        const int64_t e = tok * S + s;
        if (edge_u[e] >= 0) M = fmaxf(M, lse_part[e * rpe + r] + sp_logw(mode, w ? w[e] : 1.f));
      }
    }
    M = wave_max(M);
  }
  float den = 0.f;
  float acc[SpRow16<T>::EPL];
#pragma unroll
  for (int x = 0; x < SpRow16<T>::EPL; ++x) acc[x] = 0.f;
  for (int s0 = 0; s0 < S; s0 += 64) {
    const int s = s0 + lane;
    float a = 0.f;
    if (s < S) {
      const int64_t e = tok * S + s;
      if (edge_u[e] >= 0) {
        if (mode == 0) a = w[e];
        else if (M > -INFINITY) a = exp2f(lse_part[e * rpe + r] + sp_logw(mode, w ? w[e] : 1.f) - M);
      }
    }
    den += a;
    sp_slot_sum(o_part, tok, S, rpe, r, a, s0, lane, acc);
  }
  sp_groups_sum<T>(acc);
  float inv = 1.f;
  if (mode != 0) {
    den = wave_sum(den);
    inv = den > 0.f ? 1.f / den : 0.f;
    if (lane == 0) lse_joint[row] = den > 0.f ? M + log2f(den) : INFINITY;
  }
  sp_row_store(out + ((int64_t)tok * HQ + hq_off + r) * kSpDh, acc, inv, lane);
}

// The same combine for few rows of at most 4 * kCombSmallPerGroup slots (decode: the shared
// chapter + 64 routed), with every load of a row in one round: each lane reads the slot values
// of slots lane and lane + 64, and the partial rows go out as 16-byte loads (a row of 64 dims is
// LPR lanes: 8 for bf16, 16 for f32; lane group sg = lane / LPR reads slots sg, sg + NG, ...),
// all of them issued before any is weighted.  Right after the decode kernel has written them,
// 16-byte loads take half the time of 8-byte ones (6 against 12 us at 64 x 12 rows of 65 slots).
// The rows of skipped slots lie inside o_part but were never written: their values are dropped
// by a select (never multiplied by a zero weight, which would keep a NaN).
constexpr int kCombSmallPerGroup = 17;

template <typename T>
__global__ __launch_bounds__(64 * kCombWaves) void sparse_combine_small_kernel(
    const T* __restrict__ o_part, const float* __restrict__ lse_part, const int32_t* __restrict__ edge_u,
    const float* __restrict__ w, int mode, int S, int rpe, int64_t ntok, int HQ, int hq_off, T* __restrict__ out,
    float* __restrict__ lse_joint) {
  constexpr int EPL = SpRow16<T>::EPL, LPR = SpRow16<T>::LPR, NG = SpRow16<T>::NG;
  constexpr int NL = (4 * kCombSmallPerGroup + NG - 1) / NG;
  typedef typename SpRow16<T>::V V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kCombWaves + (threadIdx.x >> 6);
  if (row >= ntok * rpe) return;
  const int64_t tok = row / rpe;
  const int r = (int)(row % rpe);
  const int sg = lane / LPR, ch = lane % LPR;
  // slot values (lane s holds slot s and s + 64); the slot's id, lse and weight are loaded
  // together for every slot in range (the buffers hold every (token, slot, row) entry) and the
  // skipped slots masked afterwards, so they take one round of memory latency, not two
  float lg[2];
  bool ok[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int sl = lane + 64 * q;
    const int64_t e = tok * S + sl;
    const bool in = sl < S;
    const int eu = in ? edge_u[e] : -1;
    const float lp = in && mode != 0 ? lse_part[e * rpe + r] : 0.f;
    const float we = in && w ? w[e] : 1.f;
    ok[q] = in && eu >= 0;
    lg[q] = !ok[q] ? 0.f : mode == 0 ? we : lp + sp_logw(mode, we);
  }
  // partial rows of this lane group's slots, all in flight
  V v[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int j = NG * i + sg;
    v[i] = j < S ? *reinterpret_cast<const V*>(o_part + ((tok * S + j) * rpe + r) * kSpDh + EPL * ch) : V{};
  }
  float M = -INFINITY;
  if (mode != 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (ok[q]) M = fmaxf(M, lg[q]);
    M = wave_max(M);
  }
  float a[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) a[q] = !ok[q] ? 0.f : mode == 0 ? lg[q] : (M > -INFINITY ? exp2f(lg[q] - M) : 0.f);
  float acc[EPL];
#pragma unroll
  for (int x = 0; x < EPL; ++x) acc[x] = 0.f;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int j = NG * i + sg;                 // j < 64 exactly when NG * i < 64: uniform over the wave
    const float aj = __shfl(NG * i < 64 ? a[0] : a[1], j & 63, 64);
    if (j < S && aj != 0.f) {
#pragma unroll
      for (int x = 0; x < EPL; ++x) acc[x] += aj * (float)v[i][x];
    }
  }
  sp_groups_sum<T>(acc);
  float inv = 1.f;
  if (mode != 0) {
    const float den = wave_sum(a[0] + a[1]);
    inv = den > 0.f ? 1.f / den : 0.f;
    if (lane == 0) lse_joint[row] = den > 0.f ? M + log2f(den) : INFINITY;
  }
  sp_row_store(out + ((int64_t)tok * HQ + hq_off + r) * kSpDh, acc, inv, lane);
}

// ----------------------------------------------------------------- backward
// mode 0: dwe[e*rpe + r] = dO_row . o_part[e, r]      (dL/dw_s partial per head)
// else:   delta[row]     = dO_row . out_row
template <typename T>
__global__ __launch_bounds__(256) void sparse_bwd_prep_kernel(const T* __restrict__ dout, const T* __restrict__ out,
                                                              const T* __restrict__ o_part,
                                                              const int32_t* __restrict__ edge_u, int mode, int S,
                                                              int rpe, int64_t ntok, int HQ, int hq_off,
                                                              float* __restrict__ dst) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (row >= ntok * rpe) return;
  const int64_t tok = row / rpe;
  const int r = (int)(row % rpe);
  const size_t off = ((size_t)tok * HQ + hq_off + r) * kSpDh + 4 * sub;
  float d[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) d[x] = to_f(dout[off + x]);
  if (mode == 0) {
    for (int s = 0; s < S; ++s) {
      const int64_t e = tok * S + s;
      float acc = 0.f;
      if (edge_u[e] >= 0) {
        const f32x4 o = part_load4(o_part + ((size_t)e * rpe + r) * kSpDh + 4 * sub);
        acc = d[0] * o[0] + d[1] * o[1] + d[2] * o[2] + d[3] * o[3];
      }
#pragma unroll
      for (int sh = 8; sh >= 1; sh >>= 1) acc += __shfl_xor(acc, sh, 16);
      if (sub == 0) dst[(size_t)e * rpe + r] = acc;
    }
  } else {
    float acc = 0.f;
#pragma unroll
    for (int x = 0; x < 4; ++x) acc += d[x] * to_f(out[off + x]);
#pragma unroll
    for (int sh = 8; sh >= 1; sh >>= 1) acc += __shfl_xor(acc, sh, 16);
    if (sub == 0) dst[row] = acc;
  }
}

// Chapter-centric backward.  Per 32-row block of a wave: S = Q K^T and dPu = dO V^T
// (lane = key column), P from the saved log-sum-exp, dS, then
//   dV += P'^T dO, dK += scale dS^T Q         (A = row-key fragments, B = [dim][row] LDS)
//   dq_part = scale dS K                     (dS transposed through LDS)
//   dlog (modes 2-3) = row sums of dS
template <typename T>
__global__ __launch_bounds__(64 * SpCfg<T>::NW, 1) void sparse_bwd_kernel(
    const T* __restrict__ q, const T* __restrict__ dout, int HQ, const T* __restrict__ k, const T* __restrict__ v,
    int64_t cs, int64_t hs, int64_t rs, int HK, const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq,
    const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge, int S, int hk0, int hq_off, int rpe,
    int mode, const float* __restrict__ lse_row, float* __restrict__ delta_row, const float* __restrict__ w,
    float scale_log2, float scale, T* __restrict__ dk, T* __restrict__ dv, int64_t ocs, int64_t ohs, int64_t ors,
    T* __restrict__ dq_part, float* __restrict__ dlog) {
  typedef typename Frag<T>::type F8;
  constexpr int NW = SpCfg<T>::NW, NT = 64 * NW;
  using Tile = SwzTile<T, 64>;   // [key][dim] and [dim][key] tiles
  constexpr int TB = 64 * 64 * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) char sK[TB];
  __shared__ __attribute__((aligned(16))) char sV[TB];
  __shared__ __attribute__((aligned(16))) char sKt[TB];
  // per wave: Q^T, dO^T as [64 dims][32 rows] (row pitch P32) and dS as [32 rows][64 keys] (pitch PK)
  constexpr int P32 = 36, PK = 72;
  constexpr int WB = (64 * P32 > 32 * PK ? 64 * P32 : 32 * PK) * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) char sW[NW][3][WB];
  const int u = blockIdx.x, hk = hk0 + blockIdx.y;
  if (u >= n_uniq[0]) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int gid = uniq[u];
  sp_load_tile<T, NT>(sK, k + gid * cs + hk * hs, rs, tid, false);
  sp_load_tile<T, NT>(sKt, k + gid * cs + hk * hs, rs, tid, true);
  sp_load_tile<T, NT>(sV, v + gid * cs + hk * hs, rs, tid, false);
  __syncthreads();
  T* sQt = reinterpret_cast<T*>(sW[wave][0]);
  T* sDt = reinterpret_cast<T*>(sW[wave][1]);
  T* sDS = reinterpret_cast<T*>(sW[wave][2]);
  static_assert(NW * 3 * WB >= 64 * 64 * 4, "reduction buffer");

  f32x4 dka[4][4], dva[4][4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      dka[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      dva[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  const int G = HQ / HK;
  const int p0 = csr_off[u], p1 = csr_off[u + 1];
  const int nrows = (p1 - p0) * G;
  for (int r0 = 32 * wave; r0 < nrows; r0 += 32 * NW) {
    // ---- row bookkeeping (A-operand rows: lane row 16*qb + c16)
    F8 qa[2][2], da[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int r = r0 + 16 * qb + c16;
      if (r < nrows) {
        const int e = csr_edge[p0 + r / G];
        const int hq = hk * G + r % G;
        const size_t off = ((size_t)(e / S) * HQ + hq) * kSpDh;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          qa[qb][ks] = Load8<T, T>::run(q + off + 32 * ks + 8 * g);
          da[qb][ks] = Load8<T, T>::run(dout + off + 32 * ks + 8 * g);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) { qa[qb][ks] = zero_frag<T>(); da[qb][ks] = zero_frag<T>(); }
      }
    }
    // ---- stage Q^T and dO^T of the 32 rows: lane -> row (lane & 31), dims 32*(lane>>5) ..
    {
      const int rr = lane & 31, half = lane >> 5;
      const int r = r0 + rr;
      const bool ok = r < nrows;
      size_t off = 0;
      if (ok) {
        const int e = csr_edge[p0 + r / G];
        off = ((size_t)(e / S) * HQ + hk * G + r % G) * kSpDh + 32 * half;
      }
      constexpr int EPC = 16 / (int)sizeof(T);
#pragma unroll
      for (int c = 0; c < 32 / EPC; ++c) {
        V16 vq = ok ? ld16(q + off + c * EPC) : V16{{0u, 0u, 0u, 0u}};
        V16 vd = ok ? ld16(dout + off + c * EPC) : V16{{0u, 0u, 0u, 0u}};
        const T* tq = reinterpret_cast<const T*>(&vq);
        const T* td = reinterpret_cast<const T*>(&vd);
#pragma unroll
        for (int x = 0; x < EPC; ++x) {
          const int dd = 32 * half + c * EPC + x;
          sQt[dd * P32 + rr] = tq[x];
          sDt[dd * P32 + rr] = td[x];
        }
      }
    }
    // ---- per-lane row stats for rows 4g + x of block qb (C-layout rows)
    float lr[2][4], dr[2][4], wr[2][4], lw[2][4];
    int er[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int r = r0 + 16 * qb + 4 * g + x;
        er[qb][x] = -1;
        lr[qb][x] = INFINITY;
        dr[qb][x] = 0.f;
        wr[qb][x] = 1.f;
        lw[qb][x] = 0.f;
        if (r < nrows) {
          const int e = csr_edge[p0 + r / G];
          const int hq = hk * G + r % G;
          const int erw = e * rpe + (hq - hq_off);
          er[qb][x] = erw;
          if (mode == 0) {
            lr[qb][x] = lse_row[erw];
            wr[qb][x] = w[e];
          } else {
            const int64_t trow = (int64_t)(e / S) * rpe + (hq - hq_off);
            lr[qb][x] = lse_row[trow];
            dr[qb][x] = delta_row[trow];
            lw[qb][x] = sp_logw(mode, w ? w[e] : 1.f);
          }
        }
      }
    // ---- S and dPu
    f32x4 sc[2][4], dp[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        F8 kf = Tile::frag(sK, 16 * kb + c16, 32 * ks + 8 * g);
        F8 vf = Tile::frag(sV, 16 * kb + c16, 32 * ks + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          mma(sc[qb][kb], qa[qb][ks], kf);
          mma(dp[qb][kb], da[qb][ks], vf);
        }
      }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int x = 0; x < 4; ++x) sc[qb][kb][x] = exp2f(sc[qb][kb][x] * scale_log2 + lw[qb][x] - lr[qb][x]);
    if (mode == 0) {
      // per-chapter softmax delta of each row (sum over the 64 keys of P dPu), also the
      // per edge-row dO . o_s that moc_sparse_dw sums into dw
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          float t = 0.f;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) t += sc[qb][kb][x] * dp[qb][kb][x];
          t += __shfl_xor(t, 1, 16);
          t += __shfl_xor(t, 2, 16);
          t += __shfl_xor(t, 4, 16);
          t += __shfl_xor(t, 8, 16);
          dr[qb][x] = t;
          if (c16 == 0 && er[qb][x] >= 0) delta_row[er[qb][x]] = t;
        }
    }
    F8 pa[4], sa[4];
    float rowsum[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) rowsum[qb][x] = 0.f;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const float p = sc[qb][kb][x];
          float ds, pv;
          if (mode == 0) {
            ds = wr[qb][x] * p * (dp[qb][kb][x] - dr[qb][x]);
            pv = wr[qb][x] * p;
          } else {
            ds = p * (dp[qb][kb][x] - dr[qb][x]);
            pv = p;
          }
          rowsum[qb][x] += ds;
          pa[kb][4 * qb + x] = from_f<T>(pv);
          sa[kb][4 * qb + x] = from_f<T>(ds * scale);
          sDS[(16 * qb + 4 * g + x) * PK + 16 * kb + c16] = from_f<T>(ds);
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- dV, dK
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      F8 bq, bd;
      const int dd = 16 * db + c16;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        bq[x] = sQt[dd * P32 + 4 * g + x];
        bq[4 + x] = sQt[dd * P32 + 16 + 4 * g + x];
        bd[x] = sDt[dd * P32 + 4 * g + x];
        bd[4 + x] = sDt[dd * P32 + 16 + 4 * g + x];
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        mma(dva[kb][db], pa[kb], bd);
        mma(dka[kb][db], sa[kb], bq);
      }
    }
    // ---- dq_part = scale * dS K : A = dS rows from LDS (row = 16*qb + c16, keys 32*ks + 8*g ..)
    f32x4 dqa[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < 4; ++db) dqa[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      F8 as[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 8; ++x) as[qb][x] = sDS[(16 * qb + c16) * PK + 32 * ks + 8 * g + x];
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        F8 bk = Tile::frag(sKt, 16 * db + c16, 32 * ks + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) mma(dqa[qb][db], as[qb], bk);
      }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        if (er[qb][x] < 0) continue;
        T* dst = dq_part + (size_t)er[qb][x] * kSpDh;
#pragma unroll
        for (int db = 0; db < 4; ++db) dst[16 * db + c16] = from_f<T>(dqa[qb][db][x] * scale);
      }
    if (dlog) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          float s = rowsum[qb][x];
          s += __shfl_xor(s, 1, 16);
          s += __shfl_xor(s, 2, 16);
          s += __shfl_xor(s, 4, 16);
          s += __shfl_xor(s, 8, 16);
          if (c16 == 0 && er[qb][x] >= 0) dlog[er[qb][x]] = s;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // ---- cross-wave reduction of dK / dV and strided store
  __syncthreads();
  float* buf = reinterpret_cast<float*>(&sW[0][0][0]);  // NW * 3 * TB/2 bytes >= 16 KB
  T* dkb = dk + gid * ocs + hk * ohs;
  T* dvb = dv + gid * ocs + hk * ohs;
  auto reduce_store = [&](f32x4 (&acc)[4][4], T* dst) {
    for (int src = 1; src < NW; ++src) {
      if (wave == src) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int x = 0; x < 4; ++x) buf[(16 * kb + 4 * g + x) * 64 + 16 * db + c16] = acc[kb][db][x];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int x = 0; x < 4; ++x) acc[kb][db][x] += buf[(16 * kb + 4 * g + x) * 64 + 16 * db + c16];
      }
      __syncthreads();
    }
    if (wave == 0) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int x = 0; x < 4; ++x) dst[(16 * kb + 4 * g + x) * ors + 16 * db + c16] = from_f<T>(acc[kb][db][x]);
    }
  };
  reduce_store(dka, dkb);
  reduce_store(dva, dvb);
}

// dq[token, hq_off + r] = sum over valid slots of dq_part[e, r]  (one wave per row)
template <typename T>
__global__ __launch_bounds__(64 * kCombWaves) void sparse_dq_combine_kernel(const T* __restrict__ dq_part,
                                                                            const int32_t* __restrict__ edge_u, int S,
                                                                            int rpe, int64_t ntok, int HQ, int hq_off,
                                                                            T* __restrict__ dq) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kCombWaves + (threadIdx.x >> 6);
  if (row >= ntok * rpe) return;
  const int64_t tok = row / rpe;
  const int r = (int)(row % rpe);
  float acc[SpRow16<T>::EPL];
#pragma unroll
  for (int x = 0; x < SpRow16<T>::EPL; ++x) acc[x] = 0.f;
  for (int s0 = 0; s0 < S; s0 += 64) {
    const int s = s0 + lane;
    const float a = (s < S && edge_u[tok * S + s] >= 0) ? 1.f : 0.f;
    sp_slot_sum(dq_part, tok, S, rpe, r, a, s0, lane, acc);
  }
  sp_groups_sum<T>(acc);
  sp_row_store(dq + ((int64_t)tok * HQ + hq_off + r) * kSpDh, acc, 1.f, lane);
}

// dw[e] for an edge e = token * S + s, summed over its rpe rows:
//   mode 0: sum_r dwe[e, r]; modes 2/3: sum_r dlog[e, r] * d log(w) / dw.
__global__ void sparse_dw_kernel(const float* __restrict__ src, const float* __restrict__ w,
                                 const int32_t* __restrict__ edge_u, int mode, int rpe, int64_t E,
                                 float* __restrict__ dw) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float s = 0.f;
  if (edge_u[e] >= 0)
    for (int r = 0; r < rpe; ++r) s += src[(size_t)e * rpe + r];
  if (mode == 2) s = w[e] > 0.f ? s / w[e] : 0.f;
  if (mode == 3) s = w[e] > 1e-20f ? s / w[e] : 0.f;
  dw[e] = s;
}

// ----------------------------------------------------- bf16: one wave per unit
// A unit is one (distinct chapter, kv head) pair; a chapter serves ~E / n_chapters
// query rows (tens), so one wave holds the whole unit: no workgroup barriers, no
// cross-wave reduction.  Workgroups carry kUnitWaves independent waves.
// Operands that need the other orientation come from LDS through transposing reads
// (tr_frag_mk): V^T in the forward, Q^T / dO^T / K^T / dS^T in the backward.
constexpr int kUnitWaves = 4;

// [64 keys][32 query rows] bf16 (64-byte rows), 16-byte chunks XOR-swizzled by key / 4
struct DsTile {
  __device__ static __forceinline__ int off(int row, int col) {
    return row * 64 + ((((col >> 3) ^ (row >> 2)) & 3) << 4) + ((col & 7) << 1);
  }
};

struct UnitRows {
  int u, hk, gid, p0, nrows;
};

// The grid never exceeds max_u * nhk units, so u < max_u and the plan reads below are in
// bounds before the n_uniq check; issuing them together saves a dependent round trip.
__device__ __forceinline__ bool unit_setup(UnitRows& ur, const int32_t* uniq, const int32_t* n_uniq,
                                           const int32_t* csr_off, int hk0, int nhk, int G, int64_t max_u) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t unit = (int64_t)blockIdx.x * kUnitWaves + wave;
  ur.u = (int)(unit / nhk);
  if (ur.u >= max_u) return false;
  const int nu = n_uniq[0];
  ur.hk = hk0 + (int)(unit % nhk);
  ur.gid = uniq[ur.u];
  ur.p0 = csr_off[ur.u];
  ur.nrows = (csr_off[ur.u + 1] - ur.p0) * G;
  return ur.u < nu;
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes at voff of the
// buffer land at LDS address m0 + 16 l.  Inline assembly, so the wait on these loads is the
// explicit vmcnt(0) below (the compiler's own waits cover only its loads; they stay correct since
// waiting for an older load with newer DMAs outstanding only waits longer).
typedef __attribute__((address_space(3))) void* unit_lds_ptr_t;
// a value the compiler cannot see through, kept in a VGPR (a buffer load's offset, so that a
// load of a uniform value still goes out as a vector load)
__device__ __forceinline__ int wave_opaque_i(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sp_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ void unit_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, const char* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(unit_lds_ptr_t)lds;
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(m0) : "memory");
}

// Forward of one unit: S^T = K Q^T (lane = query row), per-row softmax over the chapter's 64 keys,
// O^T = V^T P^T, normalised partial rows and their lse.  The V tile goes global -> LDS by DMA (no
// registers held while it is in flight; the source addresses carry the tile's chunk swizzle), K
// fragments straight into registers, and the first 16-row block's edge ids before both, so its
// q loads go out while the tiles are in flight.  Rows are taken 16 at a time (a decode unit has
// one or two).
__global__ __launch_bounds__(64 * kUnitWaves) void sparse_fwd_unit_kernel(
    const bf16* __restrict__ q, int HQ, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t cs,
    int64_t hs, int64_t rs, int HK, const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq,
    const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge, int64_t max_u, int S, int hk0,
    int nhk, int hq_off, int rpe, float scale_log2, bf16* __restrict__ o_part, float* __restrict__ lse_part,
    const float* __restrict__ omega, const int32_t* __restrict__ row_tab) {
  using Tile = SwzTile<bf16, 64>;
  __shared__ __attribute__((aligned(1024))) char sVall[kUnitWaves][64 * 64 * 2];
  const int G = HQ / HK;
  UnitRows ur;
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  // with a row table (first 16 edges of every distinct chapter, -1 padded: the decode path,
  // whose plan is fixed for a whole generation) the first block's edge ids do not wait for
  // csr_off: they are requested together with the plan entries
  int eid_tab = -1;
  if (row_tab) {
    const int64_t u0 = ((int64_t)blockIdx.x * kUnitWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) / nhk;
    if (u0 < max_u) eid_tab = row_tab[u0 * 16 + c16 / G];
  }
  if (!unit_setup(ur, uniq, n_uniq, csr_off, hk0, nhk, G, max_u)) return;
  char* sV = sVall[threadIdx.x >> 6];
  const int64_t kv0 = (int64_t)ur.gid * cs + (int64_t)ur.hk * hs;
  {
    // DMA instruction i fills LDS rows 8 i .. 8 i + 7: lane l -> row 8 i + l / 8, physical chunk
    // l % 8 = logical chunk (l % 8) ^ (row & 7) of Tile::off
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(v + kv0), (short)0, (int)((63 * rs + 64) * 2), 0x00020000);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 8 * i + (lane >> 3), lch = (lane & 7) ^ (row & 7);
      unit_dma16(vr, (uint32_t)((row * rs + 8 * lch) * 2), sV + 1024 * i);
    }
  }
  int eid = -1;
  auto row_edge = [&](int r0) {
    const int r = r0 + c16;
    eid = r < ur.nrows ? (row_tab && r0 == 0 ? eid_tab : csr_edge[ur.p0 + r / G]) : -1;
  };
  bf16x8 qf[2];
  int erow;
  float wrow;
  auto row_operands = [&](int r0) {
    const int r = r0 + c16;
    erow = -1;
    wrow = 1.f;
    qf[0] = qf[1] = zero_frag<bf16>();
    if (eid >= 0) {
      const int hq = ur.hk * G + r % G;
      erow = eid * rpe + (hq - hq_off);
      if (omega) wrow = omega[eid];
      const bf16* qp = q + ((int64_t)(eid / S) * HQ + hq) * kSpDh + 8 * g;
      qf[0] = Load8<bf16, bf16>::run(qp);
      qf[1] = Load8<bf16, bf16>::run(qp + 32);
    }
  };
  row_edge(0);
  // K as the A operand of S^T = K Q^T (lane = key)
  bf16x8 kf[4][2];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) kf[kb][ks] = Load8<bf16, bf16>::run(k + kv0 + (16 * kb + c16) * rs + 32 * ks + 8 * g);
  row_operands(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the V tile (and everything before) has landed
  for (int r0 = 0; r0 < ur.nrows; r0 += 16) {
    if (r0 > 0) {
      row_edge(r0);
      row_operands(r0);
    }
    // S^T: lane = query row r0 + c16, keys 16 kb + 4 g + x
    f32x4 st[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      st[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma(st[kb], kf[kb][0], qf[0]);
      mma(st[kb], kf[kb][1], qf[1]);
    }
    bf16x8 pf[2];
    float mx = st[0][0];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int x = 0; x < 4; ++x) mx = fmax_fast(mx, st[kb][x]);
    const float c = wrow * scale_log2;
    const float m = quad_max(mx) * c;
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const float p = exp2f(st[kb][x] * c - m);
        ps += p;
        pf[kb >> 1][4 * (kb & 1) + x] = (bf16)p;
      }
    const float l = quad_sum(ps);
    // O^T = V^T P^T: lane = query row, dims 16 db + 4 g + x
    f32x4 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const bf16x8 a0 = tr_frag_mk<Tile>(sV, 0, 16 * db, lane);
      const bf16x8 a1 = tr_frag_mk<Tile>(sV, 32, 16 * db, lane);
      o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma(o[db], a0, pf[0]);
      mma(o[db], a1, pf[1]);
    }
    if (erow >= 0) {
      const float inv = wrow / l;
      bf16* op = o_part + (int64_t)erow * kSpDh;
#pragma unroll
      for (int db = 0; db < 4; ++db) part_store4(op + 16 * db + 4 * g, o[db] * inv);
      if (g == 0) lse_part[erow] = m + log2f(l);
    }
  }
}

// Backward of one unit on a workgroup of two waves, wave w owning keys 32 w .. 32 w + 31
// (K / V fragments and the dK / dV accumulators split in half, so two units fit per
// SIMD).  Per 32-row block: S = Q K^T and dPu = dO V^T with lane = key (accumulator
// layout, rows 16 qb + 4 g + x), P and dS in registers, then
//   dV^T += dO^T P,  dK^T += Q^T dS      (A = transposing reads of the staged rows)
//   dQ^T  = K^T dS^T over all 64 keys     (wave w: dims 32 w .. 32 w + 31)
// with the per-row sums over the chapter's 64 keys (mode 0 softmax delta sum_j P_j dPu_j,
// the d log-weight row sums of modes 2-3) added from the two waves' halves in a fixed
// order.  mode 0 writes the delta to delta_row (the per edge-row dO . o_s that
// moc_sparse_dw sums into dw).
constexpr int kBwdWaves = 2;

__global__ __launch_bounds__(64 * kBwdWaves) void sparse_bwd_unit_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ dout, int HQ, const bf16* __restrict__ k,
    const bf16* __restrict__ v, int64_t cs, int64_t hs, int64_t rs, int HK, const int32_t* __restrict__ uniq,
    const int32_t* __restrict__ n_uniq, const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge,
    int64_t max_u, int S, int hk0, int nhk, int hq_off, int rpe, int mode, const float* __restrict__ lse_row,
    float* __restrict__ delta_row, const float* __restrict__ w, float scale_log2, float scale, bf16* __restrict__ dk,
    bf16* __restrict__ dv, int64_t ocs, int64_t ohs, int64_t ors, bf16* __restrict__ dq_part,
    float* __restrict__ dlog, const int32_t* __restrict__ row_tab, uint32_t qbytes) {
  using Tile = SwzTile<bf16, 64>;
  constexpr int kKB = 64 * 64 * 2, kRB = 32 * 64 * 2;
  __shared__ __attribute__((aligned(1024))) char sK[kKB];   // K [key][dim]
  __shared__ __attribute__((aligned(1024))) char sV[kKB];   // V [key][dim]
  __shared__ __attribute__((aligned(1024))) char sQ[kRB];   // Q rows of the block [row][dim]
  __shared__ __attribute__((aligned(1024))) char sD[kRB];   // dO rows
  __shared__ __attribute__((aligned(16))) char sDS[kRB];    // dS [key][row] (DsTile)
  __shared__ __attribute__((aligned(1024))) char sDQ[kRB];  // the block's dQ rows [row][dim]
  __shared__ float sLse[32], sDel[32], sWr[32], sPart[kBwdWaves][2][32];
  __shared__ int sEr[32];
  const int G = HQ / HK;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  const int key0 = 32 * wave;
  // 16-byte LDS DMA geometry: an instruction fills 8 rows of 128 B; lane l -> row 8 i + l / 8,
  // physical chunk l % 8, which holds logical chunk (l % 8) ^ (row & 7) of Tile::off
  const int dlc = (lane & 7) ^ (lane >> 3);
  // units of the plan's distinct chapters; the workgroups walk them persistently (unit, + grid, ...)
  const int64_t lim = min((int64_t)n_uniq[0], max_u) * nhk;
  // A unit's plan entries and, with a row table (the first 32 edges of every distinct chapter),
  // its first block's edge ids, requested one unit ahead -- right after the current unit's first
  // wait -- so that a unit's first loads depend on nothing still in flight.  They go out as
  // vector loads (counted in vmcnt, which the unit's DMA wait covers anyway) rather than scalar
  // loads, whose lgkmcnt the waits on LDS reads share.  Per lane: the two rows its DMA
  // instructions move (16 wave + 8 i + lane / 8) and the constants' row lane & 31.
  struct Ahead {
    int gid, p0, p1, d0, d1, c;
  };
  auto request = [&](int64_t unit) {
    Ahead a{0, 0, 0, -1, -1, -1};
    if (unit < lim) {
      const int u = (int)(unit / nhk);
      const int z = wave_opaque_i(0);
      a.gid = __builtin_amdgcn_raw_buffer_load_b32(sp_rsrc(uniq + u, 4), z, 0, 0);
      a.p0 = __builtin_amdgcn_raw_buffer_load_b32(sp_rsrc(csr_off + u, 8), z, 0, 0);
      a.p1 = __builtin_amdgcn_raw_buffer_load_b32(sp_rsrc(csr_off + u, 8), z, 4, 0);
      if (row_tab) {
        const int32_t* tb = row_tab + (int64_t)u * 32;
        a.d0 = tb[(16 * wave + (lane >> 3)) / G];
        a.d1 = tb[(16 * wave + 8 + (lane >> 3)) / G];
        a.c = tb[(lane & 31) / G];
      }
    }
    return a;
  };
  // the rows of a block (q, dO) go to LDS by DMA, wave w moving rows 16 w .. 16 w + 15; rows past
  // the unit's read from an offset past the buffer, i.e. zeros.  The per-row constants (wave 0,
  // one lane per row) are loaded into registers and staged at the block's start.
  const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(q), (short)0, (int)qbytes,
                                                                      0x00020000);
  const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(dout), (short)0,
                                                                      (int)qbytes, 0x00020000);
  Ahead cur = request(blockIdx.x), nxt = cur;
  for (int64_t unit = blockIdx.x; unit < lim; unit += gridDim.x) {
  const int hk = hk0 + (int)(unit % nhk);
  const int gid = __builtin_amdgcn_readfirstlane(cur.gid);
  const int p0 = __builtin_amdgcn_readfirstlane(cur.p0);
  const int nrows = (__builtin_amdgcn_readfirstlane(cur.p1) - p0) * G;
  const int tab_d[2] = {cur.d0, cur.d1}, tab_c = cur.c;
  const int64_t kv0 = (int64_t)gid * cs + (int64_t)hk * hs;
  __syncthreads();   // the previous unit's dK / dV rows (staged in sK / sV) have been read back
  {
    // K and V tiles -> LDS (K the B operand of S and, transposed, of dQ; V the B operand of dPu):
    // wave w moves keys 32 w .. 32 w + 31 of each
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(k + kv0), (short)0, (int)((63 * rs + 64) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(v + kv0), (short)0, (int)((63 * rs + 64) * 2), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 8 * (4 * wave + i) + (lane >> 3);
      unit_dma16(kr, (uint32_t)((key * rs + 8 * dlc) * 2), sK + 1024 * (4 * wave + i));
      unit_dma16(vr, (uint32_t)((key * rs + 8 * dlc) * 2), sV + 1024 * (4 * wave + i));
    }
  }
  f32x4 dkt[4][2], dvt[4][2];   // [db][j]: lane = key key0 + 16 j + c16, dims 16 db + 4 g + x
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dkt[db][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      dvt[db][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  float c_lse = INFINITY, c_del = 0.f, c_w = 0.f;
  int c_er = -1;
  auto fetch_rows = [&](int r0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = r0 + 16 * wave + 8 * i + (lane >> 3);
      uint32_t off = 0xFFFFFFF0u;   // >= qbytes (host check): the load returns zeros
      if (r < nrows) {
        const int e = row_tab && r0 == 0 ? tab_d[i] : csr_edge[p0 + r / G];
        const int hq = hk * G + r % G;
        off = (uint32_t)((((int64_t)(e / S) * HQ + hq) * kSpDh + 8 * dlc) * 2);
      }
      unit_dma16(qr, off, sQ + 1024 * (2 * wave + i));
      unit_dma16(dr, off, sD + 1024 * (2 * wave + i));
    }
    c_lse = INFINITY;
    c_del = c_w = 0.f;
    c_er = -1;
    const int r = r0 + (lane & 31);
    if (wave == 0 && lane < 32 && r < nrows) {
      const int e = row_tab && r0 == 0 ? tab_c : csr_edge[p0 + r / G];
      const int hr = hk * G + r % G - hq_off;
      c_er = e * rpe + hr;
      if (mode == 0) {
        c_lse = lse_row[c_er];
        c_w = w[e];
      } else {
        const int64_t trow = (int64_t)(e / S) * rpe + hr;
        c_lse = lse_row[trow];
        c_del = delta_row[trow];
        c_w = sp_logw(mode, w ? w[e] : 1.f);
      }
    }
  };
  fetch_rows(0);
  for (int r0 = 0; r0 < nrows; r0 += 32) {
    const bool two = r0 + 16 < nrows;
    if (wave == 0 && lane < 32) {
      sLse[lane] = c_lse;
      sDel[lane] = c_del;
      sWr[lane] = c_w;
      sEr[lane] = c_er;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's DMA (K at the first block, the rows)
    __syncthreads();   // (1) rows, K and the constants visible to both waves
    if (r0 == 0) nxt = request(unit + gridDim.x);
    // ---- S and dPu for this wave's keys (lane = key, rows 16 qb + 4 g + x)
    f32x4 sc[2][2], dp[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        sc[qb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[qb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 kf[2], vf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        kf[j] = Tile::frag(sK, key0 + 16 * j + c16, 32 * ks + 8 * g);
        vf[j] = Tile::frag(sV, key0 + 16 * j + c16, 32 * ks + 8 * g);
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        if (qb == 0 || two) {
          const bf16x8 qa = Tile::frag(sQ, 16 * qb + c16, 32 * ks + 8 * g);
          const bf16x8 da = Tile::frag(sD, 16 * qb + c16, 32 * ks + 8 * g);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            mma(sc[qb][j], qa, kf[j]);
            mma(dp[qb][j], da, vf[j]);
          }
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int rr = 16 * qb + 4 * g + x;
        const float lr = sLse[rr], wr = sWr[rr];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          sc[qb][j][x] = exp2f(sc[qb][j][x] * scale_log2 + (mode == 0 ? 0.f : wr) - lr);
      }
    float dr[2][4];
    if (mode == 0) {
      // per-chapter softmax delta: this wave's 32 keys, then both halves in order
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          float t = sc[qb][0][x] * dp[qb][0][x] + sc[qb][1][x] * dp[qb][1][x];
          t += __shfl_xor(t, 1, 16);
          t += __shfl_xor(t, 2, 16);
          t += __shfl_xor(t, 4, 16);
          t += __shfl_xor(t, 8, 16);
          if (c16 == 0) sPart[wave][0][16 * qb + 4 * g + x] = t;
        }
      __syncthreads();   // (2)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int rr = 16 * qb + 4 * g + x;
          dr[qb][x] = sPart[0][0][rr] + sPart[1][0][rr];
        }
      if (wave == 0 && lane < 32) {
        const int er = sEr[lane];
        if (er >= 0) delta_row[er] = sPart[0][0][lane] + sPart[1][0][lane];
      }
    } else {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) dr[qb][x] = sDel[16 * qb + 4 * g + x];
    }
    bf16x8 pa[2], sa[2];
    float rsum[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) rsum[qb][x] = 0.f;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const float wr = mode == 0 ? sWr[16 * qb + 4 * g + x] : 1.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float pw = wr * sc[qb][j][x];
          const float ds = pw * (dp[qb][j][x] - dr[qb][x]);
          rsum[qb][x] += ds;
          pa[j][4 * qb + x] = (bf16)pw;
          sa[j][4 * qb + x] = (bf16)ds;
        }
      }
    // ---- dV^T += dO^T P, dK^T += Q^T dS
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const bf16x8 ad = tr_frag_mk<Tile>(sD, 0, 16 * db, lane);
      const bf16x8 aq = tr_frag_mk<Tile>(sQ, 0, 16 * db, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        mma(dvt[db][j], ad, pa[j]);
        mma(dkt[db][j], aq, sa[j]);
      }
    }
    // ---- dS key-major for dQ, d log-weight row sums
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int key = key0 + 16 * j + c16;
      const bf16x4 lo = {sa[j][0], sa[j][1], sa[j][2], sa[j][3]};
      const bf16x4 hi = {sa[j][4], sa[j][5], sa[j][6], sa[j][7]};
      *reinterpret_cast<bf16x4*>(sDS + DsTile::off(key, 4 * g)) = lo;
      *reinterpret_cast<bf16x4*>(sDS + DsTile::off(key, 16 + 4 * g)) = hi;
    }
    if (dlog) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          float t = rsum[qb][x];
          t += __shfl_xor(t, 1, 16);
          t += __shfl_xor(t, 2, 16);
          t += __shfl_xor(t, 4, 16);
          t += __shfl_xor(t, 8, 16);
          if (c16 == 0) sPart[wave][1][16 * qb + 4 * g + x] = t;
        }
    }
    __syncthreads();   // (3) dS and the row-sum halves visible; the rows and constants are read
    if (dlog && wave == 0 && lane < 32) {
      const int er = sEr[lane];
      if (er >= 0) dlog[er] = sPart[0][1][lane] + sPart[1][1][lane];
    }
    // the next block's rows go out now (sQ / sD are no longer read in this block) and land
    // during the dQ product
    if (r0 + 32 < nrows) fetch_rows(r0 + 32);
    // ---- dQ^T = K^T dS^T for dims 32 wave .. + 31: lane = row 16 qb + c16, dims 16 db + 4 g + x
    f32x4 dq[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) dq[i][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 bs[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) bs[qb] = tr_frag_mk<DsTile>(sDS, 32 * ks, 16 * qb, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const bf16x8 ak = tr_frag_mk<Tile>(sK, 32 * ks, 32 * wave + 16 * i, lane);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          if (qb == 0 || two) mma(dq[i][qb], ak, bs[qb]);
      }
    }
    // dQ rows staged as [row][dim] in LDS, then stored as whole 128-byte rows (16 bytes per lane,
    // chunks threadIdx + 128 t: row chunk / 8, 16-byte chunk chunk % 8); the rows' edge slots are
    // read before the barrier (the next block's constants replace them after it)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f32x4 t = dq[i][qb] * scale;
        const bf16x4 b = {(bf16)t[0], (bf16)t[1], (bf16)t[2], (bf16)t[3]};
        *reinterpret_cast<bf16x4*>(sDQ + Tile::off(16 * qb + c16, 32 * wave + 16 * i + 4 * g)) = b;
      }
    int er_st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) er_st[t] = sEr[(threadIdx.x + 128 * t) >> 3];
    __syncthreads();   // (4) the block's dQ rows staged
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int cid = threadIdx.x + 128 * t, row = cid >> 3, ch = cid & 7;
      if (er_st[t] >= 0)
        *reinterpret_cast<bf16x8*>(dq_part + (int64_t)er_st[t] * kSpDh + 8 * ch) =
            *reinterpret_cast<const bf16x8*>(sDQ + Tile::off(row, 8 * ch));
    }
  }
  // ---- dK = scale (dK^T)^T, dV: the accumulators (lane = key, 4 consecutive dims each) are
  // staged as [key][dim] rows in the K / V tiles' LDS (free once both waves have finished the
  // last dQ product), then stored as whole 128-byte rows, 16 bytes per lane
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int key = key0 + 16 * j + c16;
      bf16x4 a, b;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        a[x] = (bf16)(dkt[db][j][x] * scale);
        b[x] = (bf16)dvt[db][j][x];
      }
      *reinterpret_cast<bf16x4*>(sK + Tile::off(key, 16 * db + 4 * g)) = a;
      *reinterpret_cast<bf16x4*>(sV + Tile::off(key, 16 * db + 4 * g)) = b;
    }
  // each wave reads back its own keys' rows (LDS operations of a wave complete in order)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  bf16* dkb = dk + (int64_t)gid * ocs + (int64_t)hk * ohs;
  bf16* dvb = dv + (int64_t)gid * ocs + (int64_t)hk * ohs;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = key0 + 8 * i + (lane >> 3), ch = lane & 7;
    const int64_t off = (int64_t)key * ors + 8 * ch;
    *reinterpret_cast<bf16x8*>(dkb + off) = *reinterpret_cast<const bf16x8*>(sK + Tile::off(key, 8 * ch));
    *reinterpret_cast<bf16x8*>(dvb + off) = *reinterpret_cast<const bf16x8*>(sV + Tile::off(key, 8 * ch));
  }
  cur = nxt;
  }
}

// dK / dV blocks (chapter, kv head) that no edge of a plan touched: the sparse backward
// writes every touched block whole, so zeroing only the others replaces a zero fill of the
// whole gradient.  mark[c] = 1 for the plan's chapters; one workgroup per (chapter, head).
__global__ __launch_bounds__(256) void untouched_mark_kernel(const int32_t* __restrict__ uniq,
                                                             const int32_t* __restrict__ n_uniq, int64_t max_u,
                                                             int64_t C, int32_t* __restrict__ mark) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < min((int64_t)n_uniq[0], max_u)) {
    const int c = uniq[i];
    if (c >= 0 && c < C) mark[c] = 1;
  }
}

__global__ __launch_bounds__(256) void mark_clear_kernel(int32_t* __restrict__ mark, int64_t C) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < C) mark[i] = 0;
}

template <typename T>
__global__ __launch_bounds__(256) void zero_untouched_kernel(T* __restrict__ dk, T* __restrict__ dv, int64_t cs,
                                                             int64_t hs, int64_t rs, int hk0, int nhk,
                                                             const int32_t* __restrict__ mark) {
  const int64_t c = blockIdx.x / nhk;
  const int hk = hk0 + (int)(blockIdx.x % nhk);
  if (mark[c]) return;
  constexpr int EPC = 16 / (int)sizeof(T), CPR = 64 / EPC;  // 16-byte chunks per 64-element row
  const V16 z{{0u, 0u, 0u, 0u}};
  for (int i = threadIdx.x; i < 64 * CPR; i += 256) {
    const int64_t off = c * cs + hk * hs + (int64_t)(i / CPR) * rs + (i % CPR) * EPC;
    st16(dk + off, z);
    st16(dv + off, z);
  }
}

}  // namespace moc

using namespace moc;

namespace {
// compute units of the current device (cached)
int sp_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}
// workgroups per CU of the persistent sparse backward (its LDS and registers hold four)
constexpr int kBwdPerCU = 4;
// 16-byte K/V/q fragment loads of the one-wave-per-unit kernels
bool unit_kv_aligned(const void* q, const void* k, const void* v, int64_t cs, int64_t hs, int64_t rs) {
  return ((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 && cs % 8 == 0 &&
         hs % 8 == 0 && rs % 8 == 0;
}
}  // namespace

int moc::sparse_fwd_launch(int dtype, const void* q, int HQ, const void* k, const void* v, int64_t cs, int64_t hs,
                           int64_t rs, int HK, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                           const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk, int hq_off, int rpe,
                           float scale, const float* omega, void* o_part, float* lse_part, hipStream_t stream,
                           const char* who, const int32_t* row_tab) {
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16) {
    MOC_REQUIRE(unit_kv_aligned(q, k, v, cs, hs, rs) && ((uintptr_t)o_part & 15) == 0, MOC_ERR_ARG,
                "%s: bf16 needs 16-byte aligned q/k/v/o_part and strides that are multiples of 8", who);
    const int64_t units = max_u * nhk;
    hipLaunchKernelGGL(sparse_fwd_unit_kernel, dim3((unsigned)((units + kUnitWaves - 1) / kUnitWaves)),
                       dim3(64 * kUnitWaves), 0, stream, (const bf16*)q, HQ, (const bf16*)k, (const bf16*)v, cs, hs,
                       rs, HK, uniq, n_uniq, csr_off, csr_edge, max_u, S, hk0, nhk, hq_off, rpe, sl2, (bf16*)o_part,
                       lse_part, omega, row_tab);
    return check_launch("sparse_fwd_unit_kernel");
  }
  if (dtype == MOC_F32) {
    dim3 grid((unsigned)max_u, (unsigned)nhk);
    hipLaunchKernelGGL(sparse_fwd_kernel<float>, grid, dim3(sp_threads<float>()), 0, stream, (const float*)q, HQ,
                       (const float*)k, (const float*)v, cs, hs, rs, HK, uniq, n_uniq, csr_off, csr_edge, S, hk0,
                       hq_off, rpe, sl2, (float*)o_part, lse_part, omega);
    return check_launch("sparse_fwd_kernel");
  }
  return set_error(MOC_ERR_UNSUPPORTED, "%s: dtype %d", who, dtype);
}

extern "C" {


int moc_sparse_fwd(int dtype, const void* q, int64_t ntok, int HQ, const void* k, const void* v, int64_t cs,
                   int64_t hs, int64_t rs, int HK, int Dh, const int32_t* uniq, const int32_t* n_uniq,
                   const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk,
                   int hq_off, int rpe, float scale, void* o_part, float* lse_part, hipStream_t stream) {
  MOC_REQUIRE(q && k && v && uniq && n_uniq && csr_off && csr_edge && o_part && lse_part, MOC_ERR_ARG,
              "moc_sparse_fwd: null pointer");
  MOC_REQUIRE(Dh == kSpDh, MOC_ERR_UNSUPPORTED, "moc_sparse_fwd: head_dim %d (needs 64)", Dh);
  MOC_REQUIRE(HQ > 0 && HK > 0 && HQ % HK == 0 && nhk > 0 && hk0 >= 0 && hk0 + nhk <= HK && S > 0, MOC_ERR_ARG,
              "moc_sparse_fwd: bad heads HQ=%d HK=%d hk0=%d nhk=%d", HQ, HK, hk0, nhk);
  if (max_u == 0 || ntok == 0) return MOC_OK;
  return moc::sparse_fwd_launch(dtype, q, HQ, k, v, cs, hs, rs, HK, uniq, n_uniq, csr_off, csr_edge, max_u, S, hk0,
                                nhk, hq_off, rpe, scale, nullptr, o_part, lse_part, stream, "moc_sparse_fwd");
}

int moc_sparse_combine(int dtype, const void* o_part, const float* lse_part, const int32_t* edge_u, const float* w,
                       int mode, int S, int rpe, int64_t ntok, int HQ, int hq_off, void* out, float* lse_joint,
                       hipStream_t stream) {
  MOC_REQUIRE(o_part && lse_part && edge_u && out, MOC_ERR_ARG, "moc_sparse_combine: null pointer");
  MOC_REQUIRE(mode >= 0 && mode <= 3, MOC_ERR_ARG, "moc_sparse_combine: mode %d", mode);
  MOC_REQUIRE((mode == 0 || mode >= 2) ? w != nullptr : true, MOC_ERR_ARG, "moc_sparse_combine: mode %d needs weights", mode);
  MOC_REQUIRE(mode == 0 || lse_joint, MOC_ERR_ARG, "moc_sparse_combine: joint modes need lse_joint");
  MOC_REQUIRE(((uintptr_t)o_part & 15) == 0 && ((uintptr_t)out & 15) == 0, MOC_ERR_ARG,
              "moc_sparse_combine: o_part and out must be 16-byte aligned");
  const int64_t rows = ntok * rpe;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + kCombWaves - 1) / kCombWaves));
  // few rows (decode): latency-bound, every load of a row in one round; many rows (token
  // routing over a batch): throughput-bound, the lighter streaming kernel keeps more rows resident
  const bool small = S <= 4 * kCombSmallPerGroup && rows <= 16384;
#define SC(KERN, TT)                                                                                                  \
  hipLaunchKernelGGL(KERN<TT>, grid, dim3(64 * kCombWaves), 0, stream, (const TT*)o_part, lse_part, edge_u, w, mode, S, \
                     rpe, ntok, HQ, hq_off, (TT*)out, lse_joint)
  if (dtype == MOC_BF16) {
    if (small) SC(sparse_combine_small_kernel, bf16); else SC(sparse_combine_kernel, bf16);
  } else if (dtype == MOC_F32) {
    if (small) SC(sparse_combine_small_kernel, float); else SC(sparse_combine_kernel, float);
  } else {
    return set_error(MOC_ERR_UNSUPPORTED, "moc_sparse_combine: dtype %d", dtype);
  }
#undef SC
  return check_launch("sparse_combine_kernel");
}

int moc_sparse_bwd_prep(int dtype, const void* dout, const void* out, const void* o_part, const int32_t* edge_u,
                        int mode, int S, int rpe, int64_t ntok, int HQ, int hq_off, float* dst, hipStream_t stream) {
  MOC_REQUIRE(dout && out && edge_u && dst && (mode != 0 || o_part), MOC_ERR_ARG, "moc_sparse_bwd_prep: null pointer");
  const int64_t rows = ntok * rpe;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + 15) / 16));
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(sparse_bwd_prep_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)dout, (const bf16*)out,
                       (const bf16*)o_part, edge_u, mode, S, rpe, ntok, HQ, hq_off, dst);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(sparse_bwd_prep_kernel<float>, grid, dim3(256), 0, stream, (const float*)dout,
                       (const float*)out, (const float*)o_part, edge_u, mode, S, rpe, ntok, HQ, hq_off, dst);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_sparse_bwd_prep: dtype %d", dtype);
  return check_launch("sparse_bwd_prep_kernel");
}

int moc_sparse_bwd(int dtype, const void* q, const void* dout, int64_t ntok, int HQ, const void* k, const void* v,
                   int64_t cs, int64_t hs, int64_t rs, int HK, int Dh, const int32_t* uniq, const int32_t* n_uniq,
                   const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk,
                   int hq_off, int rpe, int mode, const float* lse_row, float* delta_row, const float* w,
                   float scale, void* dk, void* dv, int64_t ocs, int64_t ohs, int64_t ors, void* dq_part,
                   float* dlog, const int32_t* row_tab, hipStream_t stream) {
  MOC_REQUIRE(q && dout && k && v && uniq && n_uniq && csr_off && csr_edge && lse_row && delta_row && dk && dv &&
                  dq_part,
              MOC_ERR_ARG, "moc_sparse_bwd: null pointer");
  MOC_REQUIRE(Dh == kSpDh, MOC_ERR_UNSUPPORTED, "moc_sparse_bwd: head_dim %d (needs 64)", Dh);
  MOC_REQUIRE(mode >= 0 && mode <= 3 && (mode == 1 || w), MOC_ERR_ARG, "moc_sparse_bwd: mode %d / weights", mode);
  MOC_REQUIRE(HQ > 0 && HK > 0 && HQ % HK == 0 && nhk > 0 && hk0 >= 0 && hk0 + nhk <= HK && S > 0, MOC_ERR_ARG,
              "moc_sparse_bwd: bad heads");
  if (max_u == 0 || ntok == 0) return MOC_OK;
  dim3 grid((unsigned)max_u, (unsigned)nhk);
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16) {
    MOC_REQUIRE(unit_kv_aligned(q, k, v, cs, hs, rs) && ((uintptr_t)dout & 15) == 0 && ((uintptr_t)dq_part & 15) == 0 &&
                    ((uintptr_t)dk & 15) == 0 && ((uintptr_t)dv & 15) == 0 && ocs % 8 == 0 && ohs % 8 == 0 &&
                    ors % 8 == 0,
                MOC_ERR_ARG,
                "moc_sparse_bwd: bf16 needs 16-byte aligned q/dout/k/v/dq_part/dk/dv and strides that are "
                "multiples of 8");
    // q / dout rows are moved by bounded buffer loads (rows past a unit read zeros from offsets
    // past the buffer)
    const int64_t qbytes = ntok * HQ * kSpDh * 2;
    MOC_REQUIRE(qbytes < ((int64_t)1 << 32) - 16, MOC_ERR_UNSUPPORTED,
                "moc_sparse_bwd: q / dout of %lld bytes (bf16 needs < 4 GiB)", (long long)qbytes);
    const int64_t units = max_u * nhk;
    const int64_t wgs = min(units, (int64_t)kBwdPerCU * sp_cus());
    hipLaunchKernelGGL(sparse_bwd_unit_kernel, dim3((unsigned)wgs), dim3(64 * kBwdWaves), 0, stream, (const bf16*)q, (const bf16*)dout, HQ, (const bf16*)k,
                       (const bf16*)v, cs, hs, rs, HK, uniq, n_uniq, csr_off, csr_edge, max_u, S, hk0, nhk, hq_off,
                       rpe, mode, lse_row, delta_row, w, sl2, scale, (bf16*)dk, (bf16*)dv, ocs, ohs, ors,
                       (bf16*)dq_part, dlog, row_tab, (uint32_t)qbytes);
    return check_launch("sparse_bwd_unit_kernel");
  } else if (dtype == MOC_F32)
    hipLaunchKernelGGL(sparse_bwd_kernel<float>, grid, dim3(sp_threads<float>()), 0, stream, (const float*)q,
                       (const float*)dout, HQ, (const float*)k, (const float*)v, cs, hs, rs, HK, uniq, n_uniq,
                       csr_off, csr_edge, S, hk0, hq_off, rpe, mode, lse_row, delta_row, w, sl2, scale, (float*)dk,
                       (float*)dv, ocs, ohs, ors, (float*)dq_part, dlog);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_sparse_bwd: dtype %d", dtype);
  return check_launch("sparse_bwd_kernel");
}

int moc_sparse_dq_combine(int dtype, const void* dq_part, const int32_t* edge_u, int S, int rpe, int64_t ntok,
                          int HQ, int hq_off, void* dq, hipStream_t stream) {
  MOC_REQUIRE(dq_part && edge_u && dq, MOC_ERR_ARG, "moc_sparse_dq_combine: null pointer");
  MOC_REQUIRE(((uintptr_t)dq_part & 15) == 0 && ((uintptr_t)dq & 15) == 0, MOC_ERR_ARG,
              "moc_sparse_dq_combine: dq_part and dq must be 16-byte aligned");
  const int64_t rows = ntok * rpe;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + kCombWaves - 1) / kCombWaves));
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(sparse_dq_combine_kernel<bf16>, grid, dim3(64 * kCombWaves), 0, stream, (const bf16*)dq_part, edge_u, S, rpe, ntok, HQ,
                       hq_off, (bf16*)dq);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(sparse_dq_combine_kernel<float>, grid, dim3(64 * kCombWaves), 0, stream, (const float*)dq_part, edge_u, S, rpe, ntok, HQ,
                       hq_off, (float*)dq);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_sparse_dq_combine: dtype %d", dtype);
  return check_launch("sparse_dq_combine_kernel");
}

int moc_sparse_dw(const float* src, const float* w, const int32_t* edge_u, int mode, int rpe, int64_t E, float* dw,
                  hipStream_t stream) {
  MOC_REQUIRE(src && edge_u && dw && (mode == 0 || w), MOC_ERR_ARG, "moc_sparse_dw: null pointer");
  MOC_REQUIRE(mode == 0 || mode == 2 || mode == 3, MOC_ERR_ARG, "moc_sparse_dw: mode %d has no weight gradient", mode);
  if (E == 0) return MOC_OK;
  hipLaunchKernelGGL(sparse_dw_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, stream, src, w, edge_u, mode,
                     rpe, E, dw);
  return check_launch("sparse_dw_kernel");
}

int moc_sparse_zero_untouched(int dtype, void* dk, void* dv, int64_t cs, int64_t hs, int64_t rs, int64_t C, int hk0,
                              int nhk, const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, int32_t* mark,
                              hipStream_t stream) {
  MOC_REQUIRE(dk && dv && uniq && n_uniq && mark, MOC_ERR_ARG, "moc_sparse_zero_untouched: null pointer");
  MOC_REQUIRE(C > 0 && C * nhk < ((int64_t)1 << 31) && hk0 >= 0 && nhk > 0 && max_u >= 0, MOC_ERR_ARG,
              "moc_sparse_zero_untouched: C=%lld hk0=%d nhk=%d", (long long)C, hk0, nhk);
  const int64_t es = dtype == MOC_F32 ? 4 : 2;
  MOC_REQUIRE(rs >= 64 && (cs * es) % 16 == 0 && (hs * es) % 16 == 0 && (rs * es) % 16 == 0 &&
                  ((uintptr_t)dk & 15) == 0 && ((uintptr_t)dv & 15) == 0,
              MOC_ERR_ARG, "moc_sparse_zero_untouched: strides and pointers must be 16-byte multiples");
  hipLaunchKernelGGL(mark_clear_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, stream, mark, C);
  if (int rc = check_launch("mark_clear_kernel")) return rc;
  if (max_u > 0) {
    hipLaunchKernelGGL(untouched_mark_kernel, dim3((unsigned)((max_u + 255) / 256)), dim3(256), 0, stream, uniq, n_uniq,
                       max_u, C, mark);
    if (int rc = check_launch("untouched_mark_kernel")) return rc;
  }
  const dim3 grid((unsigned)(C * nhk));
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(zero_untouched_kernel<bf16>, grid, dim3(256), 0, stream, (bf16*)dk, (bf16*)dv, cs, hs, rs, hk0,
                       nhk, (const int32_t*)mark);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(zero_untouched_kernel<float>, grid, dim3(256), 0, stream, (float*)dk, (float*)dv, cs, hs, rs,
                       hk0, nhk, (const int32_t*)mark);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_sparse_zero_untouched: dtype %d", dtype);
  return check_launch("zero_untouched_kernel");
}

}  // extern "C"
