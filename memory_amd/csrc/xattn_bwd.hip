// Sequence-routed memory cross-attention, backward.
//
// Notation as in xattn_fwd.hip: logits S_ij = omega_c * scale * q_i . k_j,
// P = softmax_j(S), o_i = sum_j P_ij omega_c v_j, dO = dL/do.
//   delta_i  = dO_i . o_i
//   dPu_ij   = dO_i . v_j                      (value term without omega)
//   dS_ij    = P_ij (omega_c dPu_ij - delta_i)
//   dq_i     = sum_j dS_ij omega_c scale k_j
//   dk_j     = sum over (sequence, slot) edges e selecting the chapter of
//              omega_e scale sum_i dS_ij q_i
//   dv_j     = sum_e omega_e sum_i P_ij dO_i
//   domega_e = sum_{i, j in chapter} (dS_ij scale q_i.k_j + P_ij dPu_ij)
// These are the gradients autograd produces for the reference chain
// memory * w -> k_proj/v_proj -> softmax attention
// (memory_transformer/model.py:689-692, memory_attention.py:241-243, :301-316),
// expressed per projected chapter: dk/dv are accumulated once per distinct
// chapter (chapter-centric walk over the inverted index, no atomics, fixed
// order), so the later dX = [dk dv] [Wk; Wv] GEMM runs over distinct chapters.
#include "moc_common.h"

namespace moc {

constexpr int kBThreads = 256;
constexpr int kBDh = 64;
constexpr int kBT = 64;

// Backward pre-pass, one workgroup per (64-query block, head, sequence):
//   delta[b, h, i] = dO_i . O_i
//   qt[b, h, :, i] = Q[b, i, h, :]     dot[b, h, :, i] = dO[b, i, h, :]
// Rows of delta / qt / dot have stride Lp = round_up(L, 128); padded entries are 0.
// qt / dot are optional (null: delta only); the dK/dV kernel reads its query-major
// operands transposed from the staged Q / dO tiles instead.
template <typename T>
__global__ __launch_bounds__(256) void xattn_bwd_prep_kernel(const T* __restrict__ q, const T* __restrict__ out,
                                                             const T* __restrict__ dout, int L, int Lp, int H,
                                                             float* __restrict__ delta, T* __restrict__ qt,
                                                             T* __restrict__ dot) {
  __shared__ T tq[64][66];
  __shared__ T td[64][66];
  const int q0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const bool tr = qt != nullptr;
  for (int i = tid; tr && i < 64 * 64; i += 256) {
    const int qq = i >> 6, dd = i & 63;
    const int qi = q0 + qq;
    T vq = from_f<T>(0.f), vd = from_f<T>(0.f);
    if (qi < L) {
      const size_t off = ((size_t)(b * (size_t)L + qi) * H + h) * kBDh + dd;
      vq = q[off];
      vd = dout[off];
    }
    tq[qq][dd] = vq;
    td[qq][dd] = vd;
  }
  // delta: 4 threads per query, 16 dims each
  {
    const int qq = tid >> 2, part = tid & 3;
    const int qi = q0 + qq;
    float acc = 0.f;
    if (qi < L) {
      const T* o = out + ((size_t)(b * (size_t)L + qi) * H + h) * kBDh + 16 * part;
      const T* d = dout + ((size_t)(b * (size_t)L + qi) * H + h) * kBDh + 16 * part;
#pragma unroll
      for (int x = 0; x < 16; ++x) acc += to_f(o[x]) * to_f(d[x]);
    }
    acc += __shfl_xor(acc, 1, 4);
    acc += __shfl_xor(acc, 2, 4);
    if (part == 0) delta[((size_t)b * H + h) * Lp + qi] = acc;
  }
  if (!tr) return;
  __syncthreads();
  const size_t base = ((size_t)b * H + h) * kBDh;
  for (int i = tid; i < 64 * 64; i += 256) {
    const int dd = i >> 6, qq = i & 63;
    // query axis in MFMA key order within each 32-query group (the dK/dV operands)
    qt[(base + dd) * Lp + q0 + mfma_key_pos(qq)] = tq[qq][dd];
    dot[(base + dd) * Lp + q0 + mfma_key_pos(qq)] = td[qq][dd];
  }
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes at voff (+ soff)
// of the buffer land at LDS address m0 + 16 l.  The wait on these loads is an explicit vmcnt(0).
typedef __attribute__((address_space(3))) void* bwd_lds_ptr_t;
__device__ __forceinline__ void bq_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, const char* lds,
                                         uint32_t soff = 0) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(bwd_lds_ptr_t)lds;
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0) : "memory");
}

// dq: one workgroup = 128 queries of one (sequence, head), loop over its slots.  With `out` (the
// forward's output) the pre-pass is fused: the workgroup forms delta = rowsum(dout * out) of its
// queries from the dO fragments it loads anyway and writes it (padded rows 0) for the dK/dV
// kernel; without it delta is read.
template <typename T>
__global__ __launch_bounds__(kBThreads) void xattn_bwd_dq_kernel(
    const T* __restrict__ q, const T* __restrict__ ktiles, const T* __restrict__ vtiles,
    const int32_t* __restrict__ slot_u, const float* __restrict__ omega,
    const T* __restrict__ dout, const T* __restrict__ out, const float* __restrict__ lse, float* __restrict__ delta,
    int B, int L, int H, int HK, int NS, int64_t kv_span, int64_t kv_su, int kv_sh, int kv_st, float scale_log2,
    float scale, T* __restrict__ dq) {
  typedef typename Frag<T>::type F8;
  using Tile = SwzTile<T, 64>;
  constexpr int TB = kBT * kBDh * (int)sizeof(T);
  // double-buffered K and V tiles (32 KB bf16, 64 KB fp32); the K^T operand of dQ = dS K
  // is read from the K tile with the transposing LDS read
  __shared__ __attribute__((aligned(16))) char sK[2][TB];
  __shared__ __attribute__((aligned(16))) char sV[2][TB];

  // tiles: (sequence, head) major, 128-query block minor (XCD-local chapter tiles)
  const int nqb = (L + 127) / 128;
  const int64_t t = xcd_tile((int64_t)B * H * nqb);
  if (t < 0) return;
  const int b = (int)(t / ((int64_t)H * nqb)), h = (int)((t / nqb) % H);
  const int hk = h / (H / HK);
  const int q0 = (int)(t % nqb) * 128;
  const int Lp = nqb * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;

  F8 qf[2][2], dof[2][2];
  float lse2[2], dl[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = q0 + 32 * wave + 16 * qb + c16;
    const bool ok = qi < L;
    const size_t row = ((size_t)(b * (size_t)L + qi) * H + h) * kBDh;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qf[qb][ks] = ok ? Load8<T, T>::run(q + row + 32 * ks + 8 * g) : zero_frag<T>();
      dof[qb][ks] = ok ? Load8<T, T>::run(dout + row + 32 * ks + 8 * g) : zero_frag<T>();
    }
    lse2[qb] = ok ? lse[((size_t)b * H + h) * Lp + qi] : INFINITY;
    if (out) {
      // lane (g, c16) holds dims 32 ks + 8 g .. + 7 of query c16: 16 products, then the 4 lanes
      // of the query
      float sacc = 0.f;
      if (ok) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const F8 of = Load8<T, T>::run(out + row + 32 * ks + 8 * g);
#pragma unroll
          for (int x = 0; x < 8; ++x) sacc += to_f(dof[qb][ks][x]) * to_f(of[x]);
        }
      }
      sacc += __shfl_xor(sacc, 16);
      sacc += __shfl_xor(sacc, 32);
      dl[qb] = sacc;
      if (g == 0) delta[((size_t)b * H + h) * Lp + qi] = sacc;
    } else {
      dl[qb] = ok ? delta[((size_t)b * H + h) * Lp + qi] : 0.f;
    }
  }
  f32x4 acc[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* su = slot_u + (size_t)b * NS;
  const float* om = omega + (size_t)b * NS;
  // bf16: a slot's K and V tiles go global -> LDS by DMA (no registers held while in flight):
  // 8 instructions of 1 KB (8 rows of 128 B) per tile, wave w issuing 2w and 2w + 1; lane l fills
  // row 8 j + l / 8, physical chunk l % 8 = logical chunk (l % 8) ^ (row & 7) of Tile::off.
  // fp32: through registers.
  constexpr bool kDma = sizeof(T) == 2;
  TileIO<T, kBThreads> kio, vio;
  const uint32_t nbytes = (uint32_t)(kv_span * (int64_t)sizeof(T));
  const uint32_t row_bytes = (uint32_t)(kv_st * (int)sizeof(T));
  const Buf kb(ktiles, nbytes), vb(vtiles, nbytes);
  auto tile_off = [&](int u) { return (uint32_t)(((size_t)u * kv_su + (size_t)hk * kv_sh) * sizeof(T)); };
  const uint32_t dma_v0 = (uint32_t)((16 * wave + (lane >> 3)) * row_bytes + 16 * ((lane & 7) ^ (lane >> 3)));
  auto fetch = [&](int u, int buf) {
    if constexpr (kDma) {
      const uint32_t so = tile_off(u);
      bq_dma16(kb.r, dma_v0, sK[buf] + 2048 * wave, so);
      bq_dma16(kb.r, dma_v0 + 8 * row_bytes, sK[buf] + 2048 * wave + 1024, so);
      bq_dma16(vb.r, dma_v0, sV[buf] + 2048 * wave, so);
      bq_dma16(vb.r, dma_v0 + 8 * row_bytes, sV[buf] + 2048 * wave + 1024, so);
    } else {
      kio.load_rows(kb, tile_off(u), row_bytes, tid);
      vio.load_rows(vb, tile_off(u), row_bytes, tid);
    }
  };
  int u_cur = su[0];
  if (u_cur >= 0) {
    fetch(u_cur, 0);
    if constexpr (!kDma) {
      kio.store(sK[0], tid);
      vio.store(sV[0], tid);
    }
  }
  vm_wait_all();  // Q / dO fragments (and the first tiles) have landed on every path into the loop
  __syncthreads();
  for (int s = 0; s < NS; ++s) {
    const int buf = s & 1;
    const int u_next = (s + 1 < NS) ? su[s + 1] : -1;
    // (buffer buf ^ 1 was last read in slot s - 1, which every wave has finished)
    if (u_next >= 0) fetch(u_next, buf ^ 1);
    // a slot of zero router weight has dS = 0 (its keys and values are zero): no dQ contribution;
    // below the floor kTinyOmega its contribution is O(omega), below fp32 resolution
    const float w = u_cur >= 0 ? om[s] : 0.f;
    if (w > kTinyOmega) {
      const char* sKc = sK[buf];
      const char* sVc = sV[buf];
      const float c = w * scale_log2;
      // ds * dsc = p (w dP - delta) dsc = (p wd) (dP - delta / w) with wd = w dsc = w^2 scale:
      // p wd = exp2(c s - lse + log2 wd) takes the factor in the exponent's constant, and the dP
      // accumulators start at -delta / w (the MFMA's C operand), so dS is one multiply
      const float lwd = __builtin_amdgcn_logf(w * w * scale);
      const float offc[2] = {lse2[0] - lwd, lse2[1] - lwd};
      const float iw = __builtin_amdgcn_rcpf(w);
      const f32x4 dinit[2] = {f32x4{-dl[0] * iw, -dl[0] * iw, -dl[0] * iw, -dl[0] * iw},
                              f32x4{-dl[1] * iw, -dl[1] * iw, -dl[1] * iw, -dl[1] * iw}};
      // the chapter's 64 keys in two halves of 32 (one dQ k-step each), which halves the
      // score registers and lets three waves share a SIMD
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        f32x4 st[2][2], dp[2][2];
#pragma unroll
        for (int kbl = 0; kbl < 2; ++kbl)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            st[kbl][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
            dp[kbl][qb] = dinit[qb];
          }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int kbl = 0; kbl < 2; ++kbl) {
            const int kb = 2 * kh + kbl;
            F8 ak = Tile::frag(sKc, 16 * kb + c16, 32 * ks + 8 * g);
            F8 av = Tile::frag(sVc, 16 * kb + c16, 32 * ks + 8 * g);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              mma(st[kbl][qb], ak, qf[qb][ks]);
              mma(dp[kbl][qb], av, dof[qb][ks]);
            }
          }
        }
        F8 dsf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int kbl = 0; kbl < 2; ++kbl)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float pw = __builtin_amdgcn_exp2f(st[kbl][qb][e] * c - offc[qb]);
              dsf[qb][4 * kbl + e] = from_f<T>(pw * dp[kbl][qb][e]);
            }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const F8 bk = mk_frag<Tile, T>(sKc, 32 * kh, 16 * db, lane);  // K^T, keys in MFMA key order
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) mma(acc[qb][db], dsf[qb], bk);
        }
      }
    }
    if (u_next >= 0) {
      if constexpr (kDma) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next slot's tiles landed
      } else {
        kio.store(sK[buf ^ 1], tid);
        vio.store(sV[buf ^ 1], tid);
      }
    }
    u_cur = u_next;
    __syncthreads();
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int qi = q0 + 32 * wave + 16 * qb + 4 * g + e;
      if (qi < L) {
        T* dst = dq + ((size_t)(b * (size_t)L + qi) * H + h) * kBDh;
#pragma unroll
        for (int db = 0; db < 4; ++db) dst[16 * db + c16] = from_f<T>(acc[qb][db][e]);
      }
    }
}

// dk/dv, slot-group decomposition.  One workgroup = one (sequence b, kv head hk,
// group of CPW consecutive slots); each slot's chapter (64 keys) is split over two
// waves of 32 keys, so a wave's accumulators, K / V fragments and score tiles fit in
// 256 registers and two waves share each SIMD.  A bf16 workgroup is 4 waves (2 slots),
// one per SIMD, so the two waves on a SIMD belong to different workgroups: their steps
// are not aligned by a common barrier, and one wave's MFMAs run under the other's
// softmax work (8-wave workgroups, in lockstep, measured 5% slower).  All slots of a
// sequence attend the same queries, so the query-side tiles of a step (Q and dO
// row-major, Q^T and dO^T, QS queries each) are staged in LDS once per workgroup and
// shared by its waves; they are
// double-buffered, the next step's global loads being issued before the math of the
// current one, so a step costs one barrier.  K and V fragments live in registers for
// the whole kernel (loaded once from HBM).  Output: per-edge dk / dv rows (edge e =
// b*NS + slot) and d omega per (edge, kv head).
//
// Per score element (key j, query i) with p = exp2(c s - lse_i) the softmax
// probability (c = omega * scale * log2 e, s = q_i . k_j, dP = dO_i . v_j):
//   t    = scale (omega dP - delta_i)
//   dk'_j = sum_i p t q_i      dv'_j = sum_i p dO_i     (A operands p t and p)
// The per-wave constants are folded into the register-resident operands once per kernel:
// k~ = c k and v~ = omega scale v, so the logit product Q k~^T started from the accumulator
// -lse is the exp2 argument itself and dO v~^T started from -scale delta is t; each element
// then costs one exp2, one multiply (p t) and half of two conversions (the bf16 operands
// k~, v~ carry one rounding of the scaled values, as the reference's omega-weighted memory
// does before its projection).
// dk = omega dk' and dv = omega dv' (the keys enter the logits and the values the output
// scaled by omega), applied once at the store; d omega = sum_ij (p t s + p dP) =
// sum_j dk'_j . k_j + dv'_j . v_j with the unscaled k, v, read off the accumulators, the two
// key halves summed in a fixed order.  The same loop serves omega == 0 (k~ = v~ = 0: every
// logit of the chapter 0, t = -scale delta, dk = dv = 0).
template <typename T> struct DkvCfg;
template <> struct DkvCfg<bf16> { static constexpr int CPW = 2, QS = 128; };
template <> struct DkvCfg<float> { static constexpr int CPW = 2, QS = 32; };
constexpr int kDkvWavesPerChapter = 2;

template <typename T>
__global__ __launch_bounds__(64 * kDkvWavesPerChapter * DkvCfg<T>::CPW) void xattn_bwd_dkv_kernel(
    const T* __restrict__ q, const T* __restrict__ dout,
    const T* __restrict__ ktiles, const T* __restrict__ vtiles, const int32_t* __restrict__ slot_u,
    const float* __restrict__ omega, const float* __restrict__ lse, const float* __restrict__ delta, int B, int L,
    int Lp, int H, int HK, int NS, int64_t kv_su, int kv_sh, int kv_st, float scale_log2, float scale,
    T* __restrict__ dkv_edge, float* __restrict__ domega_part) {
  typedef typename Frag<T>::type F8;
  constexpr int CPW = DkvCfg<T>::CPW, QS = DkvCfg<T>::QS;
  constexpr int WPC = kDkvWavesPerChapter, NW = CPW * WPC, NT = 64 * NW;
  constexpr int NKB = 64 / WPC / 16;              // 16-key blocks per wave
  constexpr int EPC = 16 / (int)sizeof(T);
  using TileK = SwzTile<T, 64>;   // [query][dim]
  constexpr int STB = 64 * QS * (int)sizeof(T);  // one staged tile (always 8 KB)
  constexpr int CPT = STB / 16 / NT;             // chunks per thread per staged tile
  static_assert(CPT >= 1, "staging needs at least one chunk per thread");
  __shared__ __attribute__((aligned(16))) char sStage[2][2][STB];  // [buf][Q, dO]
  __shared__ float sL[2][QS], sDl[2][QS];
  __shared__ float sDom[NW];

  // tiles: (sequence, kv head) major, slot group minor, so the slot groups that stage
  // the same query tiles share one XCD's L2
  const int nsg = (NS + CPW - 1) / CPW;
  const int64_t t = xcd_tile((int64_t)B * HK * nsg);
  if (t < 0) return;
  const int b = (int)(t / ((int64_t)HK * nsg)), hk = (int)((t / nsg) % HK);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int slot = CPW * (int)(t % nsg) + wave / WPC;
  const int k0 = 64 / WPC * (wave % WPC);  // this wave's first key of the chapter
  const int e = b * NS + slot;
  const int u = slot < NS ? slot_u[e] : -1;
  const bool active = u >= 0;
  const int G = H / HK;
  const int KV = HK * 64;
  const size_t row_stride = 2 * (size_t)KV;

  // K / V fragments of this wave's keys: B operands of S = Q K^T and dP = dO V^T
  // (key row k0 + 16 kb + c16, dims 32 ks + 8 g .. +7)
  F8 kreg[NKB][2], vreg[NKB][2];
  if (active) {
    const T* kp = ktiles + (size_t)u * kv_su + (size_t)hk * kv_sh;
    const T* vp = vtiles + (size_t)u * kv_su + (size_t)hk * kv_sh;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kreg[kb][ks] = Load8<T, T>::run(kp + (size_t)(k0 + 16 * kb + c16) * kv_st + 32 * ks + 8 * g);
        vreg[kb][ks] = Load8<T, T>::run(vp + (size_t)(k0 + 16 * kb + c16) * kv_st + 32 * ks + 8 * g);
      }
  }
  const float w = active ? omega[e] : 0.f;
  const float c = w * scale_log2, dsc = w * scale;
  // k~ = c k, v~ = omega scale v (see above)
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        kreg[kb][ks][x] = from_f<T>(c * to_f(kreg[kb][ks][x]));
        vreg[kb][ks][x] = from_f<T>(dsc * to_f(vreg[kb][ks][x]));
      }

  f32x4 dk[NKB][4], dv[NKB][4];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      dk[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      dv[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int nstep = (L + QS - 1) / QS;
  for (int hq = hk * G; hq < hk * G + G; ++hq) {
    const size_t bh = (size_t)b * H + hq;
    // staged tiles of a step: 0 = Q rows, 1 = dO rows ([query][dim]; the query-major operands
    // Q^T, dO^T of dK, dV are read from them with the transposing LDS read); every thread
    // moves CPT 16-byte chunks of each.  Rows are read through a buffer spanning this
    // sequence only, so rows past L come back as zeros.
    const uint32_t seq_bytes = (uint32_t)((size_t)L * H * 64 * sizeof(T));
    const Buf bq(q + (size_t)b * L * H * 64, seq_bytes), bd(dout + (size_t)b * L * H * 64, seq_bytes);
    uint32_t voff_r[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int r = tid + NT * j;
      const int qq = r / (64 / EPC), cc = (r % (64 / EPC)) * EPC;
      voff_r[j] = (uint32_t)(((qq * H + hq) * 64 + cc) * (int)sizeof(T));
    }
    // bf16: the Q and dO tiles go global -> LDS by DMA (buffer_load ... lds, no registers held
    // while they are in flight): a tile is STB / 1 KB instructions of 8 rows of 128 B, wave w
    // issues the IPW consecutive instructions IPW w .. of each tile; lane l fills row
    // 8 j + l / 8, physical chunk l % 8, which holds logical chunk (l % 8) ^ (row & 7) of
    // TileK::off.  fp32: through registers.
    constexpr bool kDma = sizeof(T) == 2;
    constexpr int IPW = STB / 1024 / NW;
    static_assert(!kDma || (IPW * NW * 1024 == STB && IPW >= 1), "DMA staging geometry");
    const int dlc = (lane & 7) ^ (lane >> 3);
    const uint32_t dvo0 =
        (uint32_t)((((8 * IPW * (tid >> 6) + (lane >> 3)) * H + hq) * 64 + 8 * dlc) * (int)sizeof(T));
    constexpr uint32_t kDvoRows8 = 8u * 64u * (uint32_t)sizeof(T);  // x H: 8 rows further
    V16 pre[kDma ? 1 : 2 * CPT];
    float preL = 0.f, preD = 0.f;
    auto fetch = [&](int st, int buf) {
      const int q0 = st * QS;
      const uint32_t so_r = (uint32_t)((size_t)q0 * H * 64 * sizeof(T));
      if constexpr (kDma) {
        // rows past L: the row offset rides in the per-lane offset, which the bound checks
        const char* l0 = sStage[buf][0] + 1024 * IPW * (tid >> 6);
        const char* l1 = sStage[buf][1] + 1024 * IPW * (tid >> 6);
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
          const uint32_t vo = dvo0 + so_r + (uint32_t)i * kDvoRows8 * (uint32_t)H;
          bq_dma16(bq.r, vo, l0 + 1024 * i);
          bq_dma16(bd.r, vo, l1 + 1024 * i);
        }
      } else {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
          pre[j] = bq.load16(voff_r[j], so_r);
          pre[CPT + j] = bd.load16(voff_r[j], so_r);
        }
      }
      if (tid < QS) {
        preL = lse[bh * Lp + q0 + tid];
        preD = delta[bh * Lp + q0 + tid];
      }
    };
    auto stash = [&](int buf) {
      if constexpr (!kDma) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
          const int r = tid + NT * j;
          const int qq = r / (64 / EPC), cc = (r % (64 / EPC)) * EPC;
          st16(sStage[buf][0] + TileK::off(qq, cc), pre[j]);
          st16(sStage[buf][1] + TileK::off(qq, cc), pre[CPT + j]);
        }
      }
      if (tid < QS) {
        // the accumulator starts -lse and -scale delta; negated and scaled here, not in fetch,
        // so the loads stay in flight across a step's math
        sL[buf][tid] = -preL;
        sDl[buf][tid] = -preD * scale;
      }
    };
    fetch(0, 0);
    stash(0);
    if constexpr (kDma) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int st = 0; st < nstep; ++st) {
      const int buf = st & 1;
      // (buffer buf ^ 1 was last read in step st - 1, which every wave has finished)
      if (st + 1 < nstep) fetch(st + 1, buf ^ 1);
      if (active) {
        const char* sQ = sStage[buf][0];
        const char* sD = sStage[buf][1];
#pragma unroll
        for (int half = 0; half < QS / 32; ++half) {
          const int qb0 = 32 * half;
          f32x4 sc[2][NKB], dp[2][NKB];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            // -lse and -scale delta of the tile's queries (rows 4 g + x of the accumulator)
            const f32x4 nl2 = *reinterpret_cast<const f32x4*>(&sL[buf][qb0 + 16 * qb + 4 * g]);
            const f32x4 ndl = *reinterpret_cast<const f32x4*>(&sDl[buf][qb0 + 16 * qb + 4 * g]);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
              sc[qb][kb] = nl2;
              dp[qb][kb] = ndl;
            }
          }
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            F8 qa[2], da[2];
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              qa[qb] = TileK::frag(sQ, qb0 + 16 * qb + c16, 32 * ks + 8 * g);
              da[qb] = TileK::frag(sD, qb0 + 16 * qb + c16, 32 * ks + 8 * g);
            }
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) {
                mma(sc[qb][kb], qa[qb], kreg[kb][ks]);
                mma(dp[qb][kb], da[qb], vreg[kb][ks]);
              }
          }
          F8 pa[NKB], sa[NKB];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
              for (int x = 0; x < 4; ++x) {
                const float pt = __builtin_amdgcn_exp2f(sc[qb][kb][x]);  // p = exp2(c s - lse)
                pa[kb][4 * qb + x] = from_f<T>(pt);
                sa[kb][4 * qb + x] = from_f<T>(pt * dp[qb][kb][x]);    // p scale (omega dP - delta)
              }
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            // Q^T / dO^T fragments (dims 16 db + c16, queries in MFMA key order) read
            // transposed from the row tiles
            const F8 fq = mk_frag<TileK, T>(sQ, qb0, 16 * db, lane);
            const F8 fd = mk_frag<TileK, T>(sD, qb0, 16 * db, lane);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
              mma(dv[kb][db], pa[kb], fd);
              mma(dk[kb][db], sa[kb], fq);
            }
          }
        }
      }
      if (st + 1 < nstep) stash(buf ^ 1);
      if constexpr (kDma) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next step's tiles landed
      __syncthreads();
    }
  }
  // dL/domega = sum_ij p (t s + dP) = sum_j dk'_j . k_j + dv'_j . v_j, summed over the query
  // heads of hk and, in a fixed order, over the chapter's two key halves
  float dom = 0.f;
  if (active) {
    const T* kp = ktiles + (size_t)u * kv_su + (size_t)hk * kv_sh;
    const T* vp = vtiles + (size_t)u * kv_su + (size_t)hk * kv_sh;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const size_t off = (size_t)(k0 + 16 * kb + 4 * g + x) * kv_st + 16 * db + c16;
          dom += dk[kb][db][x] * to_f(kp[off]) + dv[kb][db][x] * to_f(vp[off]);
        }
    dom = wave_sum(dom);
  }
  if (lane == 0) sDom[wave] = dom;
  __syncthreads();
  if (!active) {
    // a skipped slot's d omega is 0 (written, so the caller needs no zero fill)
    if (slot < NS && wave % WPC == 0 && lane == 0) domega_part[(size_t)e * HK + hk] = 0.f;
    return;
  }
  if (wave % WPC == 0 && lane == 0) {
    float s = 0.f;
    for (int i = 0; i < WPC; ++i) s += sDom[wave + i];
    domega_part[(size_t)e * HK + hk] = s;
  }
  T* rows = dkv_edge + (size_t)e * 64 * row_stride;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int key = k0 + 16 * kb + 4 * g + x, dim = 16 * db + c16;
        rows[(size_t)key * row_stride + hk * 64 + dim] = from_f<T>(w * dk[kb][db][x]);
        rows[(size_t)key * row_stride + KV + hk * 64 + dim] = from_f<T>(w * dv[kb][db][x]);
      }
}

// dkv[u*T + t, :] = sum over the edges of distinct chapter u (csr order) of
// dkv_edge[e*T + t, :]; zero rows for unused plan slots.  grid (max_u, kRedSplit):
// each workgroup sums one slice of the chapter block in 16-byte chunks.
constexpr int kRedSplit = 16;
template <typename T>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(const T* __restrict__ dkv_edge,
                                                         const int32_t* __restrict__ n_uniq,
                                                         const int32_t* __restrict__ csr_off,
                                                         const int32_t* __restrict__ csr_edge, int64_t row_elems,
                                                         T* __restrict__ dkv) {
  constexpr int EPC = 16 / (int)sizeof(T);
  const int u = blockIdx.x;
  const int64_t n = 64 * row_elems;     // elements of one chapter block
  const int64_t nch = n / EPC;          // 16-byte chunks
  const int64_t per = (nch + kRedSplit - 1) / kRedSplit;
  const int64_t c0 = (int64_t)blockIdx.y * per, c1 = min(nch, c0 + per);
  T* dst = dkv + (size_t)u * n;
  if (u >= n_uniq[0]) {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) st16(dst + i * EPC, V16{{0u, 0u, 0u, 0u}});
    return;
  }
  const int p0 = csr_off[u], p1 = csr_off[u + 1];
  if (p1 - p0 == 1) {
    const T* src = dkv_edge + (size_t)csr_edge[p0] * n;
    for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) st16(dst + i * EPC, ld16(src + i * EPC));
    return;
  }
  for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) {
    float acc[EPC];
#pragma unroll
    for (int x = 0; x < EPC; ++x) acc[x] = 0.f;
    for (int p = p0; p < p1; ++p) {
      V16 v = ld16(dkv_edge + (size_t)csr_edge[p] * n + i * EPC);
      const T* t = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int x = 0; x < EPC; ++x) acc[x] += to_f(t[x]);
    }
    T o[EPC];
#pragma unroll
    for (int x = 0; x < EPC; ++x) o[x] = from_f<T>(acc[x]);
    st16(dst + i * EPC, *reinterpret_cast<V16*>(o));
  }
}

// X[r, :] = norm(bank[uniq[r / T] * T + r % T, :]) in the compute dtype; rows of
// unused plan slots (r >= n_uniq * T) are zero.  One wave per row, 16-byte chunks
// (d % 8 == 0).
template <typename TO, typename TI>
__device__ __forceinline__ void load8f(const TI* p, float* o) {
  if constexpr (sizeof(TI) == 2) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int x = 0; x < 8; ++x) o[x] = (float)v[x];
  } else {
    f32x4 a = *reinterpret_cast<const f32x4*>(p), c = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int x = 0; x < 4; ++x) { o[x] = a[x]; o[4 + x] = c[x]; }
  }
}
template <typename TO>
__device__ __forceinline__ void store8f(TO* p, const float* v) {
  if constexpr (sizeof(TO) == 2) {
    bf16x8 r;
#pragma unroll
    for (int x = 0; x < 8; ++x) r[x] = (bf16)v[x];
    *reinterpret_cast<bf16x8*>(p) = r;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

template <typename T, typename TB>
__global__ __launch_bounds__(256) void gather_rows_kernel(const TB* __restrict__ bank, int64_t d, int Tc,
                                                          const int32_t* __restrict__ uniq,
                                                          const int32_t* __restrict__ n_uniq, int64_t rows,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd, T* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int64_t valid = (int64_t)n_uniq[0] * Tc;
  T* o = out + r * d;
  float v[8];
  if (r >= valid) {
#pragma unroll
    for (int x = 0; x < 8; ++x) v[x] = 0.f;
    for (int64_t j = 8 * lane; j < d; j += 512) store8f<T>(o + j, v);
    return;
  }
  const TB* xr = bank + ((int64_t)uniq[r / Tc] * Tc + r % Tc) * d;
  const float mu = rstd ? mean[r] : 0.f, rs = rstd ? rstd[r] : 1.f;
  for (int64_t j = 8 * lane; j < d; j += 512) {
    load8f<T, TB>(xr + j, v);
#pragma unroll
    for (int x = 0; x < 8; ++x) v[x] = (v[x] - mu) * rs;
    store8f<T>(o + j, v);
  }
}

// grad_bank[src(r), :] = norm_bwd(g_r) for r < n_uniq * T, where g_r is dX[r, :] (one dX row
// per distinct-chapter row) or, given the plan's inverted index, the sum over the chapter's
// edges (csr order, deterministic) of the per-edge rows dX[e * T + t, :].  Distinct chapters
// own distinct bank rows, so plain stores suffice (grad_bank must be zero-initialised by the
// caller for rows that are not selected).  With `fresh` (accumulator mode) chapter u's rows are
// stored when fresh[u] is set and added to the rows already there otherwise.
template <typename TX, typename TB, typename TG>
__global__ __launch_bounds__(256) void bank_scatter_kernel(const TX* __restrict__ dX, const TB* __restrict__ bank,
                                                           int64_t d, int Tc, const int32_t* __restrict__ uniq,
                                                           const int32_t* __restrict__ n_uniq, int64_t rows,
                                                           const int32_t* __restrict__ csr_off,
                                                           const int32_t* __restrict__ csr_edge,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd, int layernorm,
                                                           const int32_t* __restrict__ fresh,
                                                           TG* __restrict__ grad) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows || r >= (int64_t)n_uniq[0] * Tc) return;
  const int64_t u = r / Tc, t = r % Tc;
  const int64_t src = (int64_t)uniq[u] * Tc + t;
  const int p0 = csr_off ? csr_off[u] : 0, p1 = csr_off ? csr_off[u + 1] : 0;
  // gradient w.r.t. the gathered row, 8 columns starting at j
  auto grow = [&](int64_t j, float* gv) {
    if (!csr_off) {
      load8f<TG, TX>(dX + r * d + j, gv);
      return;
    }
#pragma unroll
    for (int x = 0; x < 8; ++x) gv[x] = 0.f;
    for (int p = p0; p < p1; ++p) {
      float e8[8];
      load8f<TG, TX>(dX + ((int64_t)csr_edge[p] * Tc + t) * d + j, e8);
#pragma unroll
      for (int x = 0; x < 8; ++x) gv[x] += e8[x];
    }
  };
  TG* o = grad + src * d;
  const bool add = fresh != nullptr && fresh[u] == 0;
  auto put = [&](int64_t j, float* gv) {
    if (add) {
      float old8[8];
      load8f<TG, TG>(o + j, old8);
#pragma unroll
      for (int x = 0; x < 8; ++x) gv[x] += old8[x];
    }
    store8f<TG>(o + j, gv);
  };
  float gv[8];
  if (!rstd) {
    for (int64_t j = 8 * lane; j < d; j += 512) {
      grow(j, gv);
      put(j, gv);
    }
    return;
  }
  const TB* xr = bank + src * d;
  const float mu = mean[r], rs = rstd[r];
  float sg = 0.f, sgx = 0.f, xv[8];
  for (int64_t j = 8 * lane; j < d; j += 512) {
    grow(j, gv);
    load8f<TG, TB>(xr + j, xv);
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      sg += gv[x];
      sgx += gv[x] * (xv[x] - mu) * rs;
    }
  }
  sg = wave_sum(sg) / (float)d;
  sgx = wave_sum(sgx) / (float)d;
  for (int64_t j = 8 * lane; j < d; j += 512) {
    grow(j, gv);
    load8f<TG, TB>(xr + j, xv);
#pragma unroll
    for (int x = 0; x < 8; ++x) gv[x] = rs * (gv[x] - (layernorm ? sg : 0.f) - (xv[x] - mu) * rs * sgx);
    put(j, gv);
  }
}

// fresh[u] = 1 when chapter uniq[u] has no rows in the accumulator for `epoch` yet (its tag
// differs), 0 otherwise; the tag is then set.  The plan's chapters are distinct.
__global__ __launch_bounds__(256) void bank_grad_mark_kernel(const int32_t* __restrict__ uniq,
                                                             const int32_t* __restrict__ n_uniq, int64_t max_u,
                                                             int epoch, int32_t* __restrict__ chap_epoch,
                                                             int32_t* __restrict__ fresh) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= max_u || u >= (int64_t)n_uniq[0]) return;
  const int32_t c = uniq[u];
  fresh[u] = chap_epoch[c] != epoch ? 1 : 0;
  chap_epoch[c] = epoch;
}

// Zero fill of the dense bank gradient by a few single-wave workgroups (one per CU by
// default), 4 x 16 bytes per lane per iteration.  Launched on a side stream beside the
// attention backward (the layer's dQ kernel), its waves sit beside the attention-backward
// waves (16 VGPRs, no LDS) and use HBM bandwidth those MFMA / VALU-bound kernels leave idle.  The
// stores are non-temporal (global_store ... nt), so the zeros stream past the L2s instead of
// evicting the tiles the attention kernels re-read there (c3, beside dQ: the fill 155 -> ~110 us,
// dQ 221 -> 193 us).
__global__ __launch_bounds__(64) void fill_zero_kernel(V16* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 64;
  int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4* d4 = reinterpret_cast<u32x4*>(dst);
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    __builtin_nontemporal_store(z4, d4 + i);
    __builtin_nontemporal_store(z4, d4 + i + stride);
    __builtin_nontemporal_store(z4, d4 + i + 2 * stride);
    __builtin_nontemporal_store(z4, d4 + i + 3 * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(z4, d4 + i);
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_xattn_bwd_prep(int dtype, const void* q, const void* out, const void* dout, int64_t B, int64_t L, int H,
                       int Dh, float* delta, void* qt, void* dot, hipStream_t stream) {
  MOC_REQUIRE(q && out && dout && delta && (qt != nullptr) == (dot != nullptr), MOC_ERR_ARG,
              "moc_xattn_bwd_prep: null pointer (qt and dot are both set or both null)");
  MOC_REQUIRE(Dh == kBDh, MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_prep: head_dim %d (needs 64)", Dh);
  MOC_REQUIRE(B >= 0 && L >= 0 && H > 0 && B < 65536, MOC_ERR_ARG, "moc_xattn_bwd_prep: bad shape");
  if (B == 0 || L == 0) return MOC_OK;
  const int Lp = (int)((L + 127) / 128 * 128);
  dim3 grid((unsigned)(Lp / 64), (unsigned)H, (unsigned)B);
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_bwd_prep_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)q, (const bf16*)out,
                       (const bf16*)dout, (int)L, Lp, H, delta, (bf16*)qt, (bf16*)dot);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_bwd_prep_kernel<float>, grid, dim3(256), 0, stream, (const float*)q, (const float*)out,
                       (const float*)dout, (int)L, Lp, H, delta, (float*)qt, (float*)dot);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_prep: dtype %d", dtype);
  return check_launch("xattn_bwd_prep_kernel");
}

}  // extern "C"

namespace moc {
namespace {
int bwd_dq(const char* who, int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span,
           int64_t su, int sh, int st, const int32_t* slot_u, const float* omega, const void* out, const void* dout,
           const float* lse, float* delta, int64_t B, int64_t L, int H, int HK, int Dh, int T, int NS, float scale,
           void* dq, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && slot_u && omega && dout && lse && delta && dq, MOC_ERR_ARG,
              "%s: null pointer", who);
  MOC_REQUIRE(Dh == kBDh && T == kBT, MOC_ERR_UNSUPPORTED, "%s: needs head_dim 64 and T 64", who);
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0, MOC_ERR_ARG, "%s: bad shape", who);
  if (int rc = check_kv_layout(who, dtype, kv_span, su, sh, st)) return rc;
  if (B == 0 || L == 0) return MOC_OK;
  MOC_REQUIRE(B * H * ((L + 127) / 128) < ((int64_t)1 << 31), MOC_ERR_UNSUPPORTED, "%s: grid too large", who);
  dim3 grid(xcd_grid(B * H * ((L + 127) / 128)));
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_bwd_dq_kernel<bf16>, grid, dim3(kBThreads), 0, stream, (const bf16*)q, (const bf16*)k_tiles,
                       (const bf16*)v_tiles, slot_u, omega, (const bf16*)dout, (const bf16*)out, lse, delta, (int)B,
                       (int)L, H, HK, NS, kv_span, su, sh, st, sl2, scale, (bf16*)dq);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_bwd_dq_kernel<float>, grid, dim3(kBThreads), 0, stream, (const float*)q,
                       (const float*)k_tiles, (const float*)v_tiles, slot_u, omega, (const float*)dout,
                       (const float*)out, lse, delta, (int)B, (int)L, H, HK, NS, kv_span, su, sh, st, sl2, scale,
                       (float*)dq);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "%s: dtype %d", who, dtype);
  return check_launch("xattn_bwd_dq_kernel");
}
}  // namespace
}  // namespace moc

extern "C" {

int moc_xattn_bwd_dq(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span,
                     int64_t su, int sh, int st, const int32_t* slot_u, const float* omega, const void* dout, const float* lse,
                     const float* delta, int64_t B, int64_t L, int H, int HK, int Dh, int T, int NS, float scale,
                     void* dq, hipStream_t stream) {
  return bwd_dq("moc_xattn_bwd_dq", dtype, q, k_tiles, v_tiles, kv_span, su, sh, st, slot_u, omega, nullptr, dout, lse,
                const_cast<float*>(delta), B, L, H, HK, Dh, T, NS, scale, dq, stream);
}

int moc_xattn_bwd_dq_delta(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span,
                           int64_t su, int sh, int st, const int32_t* slot_u, const float* omega, const void* out,
                           const void* dout, const float* lse, float* delta, int64_t B, int64_t L, int H, int HK, int Dh,
                           int T, int NS, float scale, void* dq, hipStream_t stream) {
  MOC_REQUIRE(out, MOC_ERR_ARG, "moc_xattn_bwd_dq_delta: null pointer");
  return bwd_dq("moc_xattn_bwd_dq_delta", dtype, q, k_tiles, v_tiles, kv_span, su, sh, st, slot_u, omega, out, dout,
                lse, delta, B, L, H, HK, Dh, T, NS, scale, dq, stream);
}

int moc_xattn_bwd_dkv(int dtype, const void* q, const void* dout,
                      const void* k_tiles, const void* v_tiles, int64_t kv_span, int64_t su, int sh, int st,
                      const int32_t* slot_u, const float* omega,
                      const float* lse, const float* delta, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                      int NS, float scale, void* dkv_edge, float* domega_part, hipStream_t stream) {
  MOC_REQUIRE(q && dout && k_tiles && v_tiles && slot_u && omega && lse && delta && dkv_edge &&
                  domega_part,
              MOC_ERR_ARG, "moc_xattn_bwd_dkv: null pointer");
  MOC_REQUIRE(Dh == kBDh && T == kBT, MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dkv: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0 && B >= 0 && B < 65536, MOC_ERR_ARG,
              "moc_xattn_bwd_dkv: bad shape");
  MOC_REQUIRE(L * H * 64 * (dtype == MOC_F32 ? 4 : 2) < ((int64_t)1 << 32), MOC_ERR_UNSUPPORTED,
              "moc_xattn_bwd_dkv: one sequence's q / dout must be < 4 GiB (L=%lld, H=%d)", (long long)L, H);
  if (int rc = check_kv_layout("moc_xattn_bwd_dkv", dtype, kv_span, su, sh, st)) return rc;
  if (B == 0 || L == 0) return MOC_OK;
  const int Lp = (int)((L + 127) / 128 * 128);
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16) {
    constexpr int CPW = DkvCfg<bf16>::CPW;
    dim3 grid(xcd_grid(B * HK * ((NS + CPW - 1) / CPW)));
    hipLaunchKernelGGL(xattn_bwd_dkv_kernel<bf16>, grid, dim3(64 * kDkvWavesPerChapter * CPW), 0, stream, (const bf16*)q,
                       (const bf16*)dout, (const bf16*)k_tiles, (const bf16*)v_tiles, slot_u,
                       omega, lse, delta, (int)B, (int)L, Lp, H, HK, NS, su, sh, st, sl2, scale, (bf16*)dkv_edge,
                       domega_part);
  } else if (dtype == MOC_F32) {
    constexpr int CPW = DkvCfg<float>::CPW;
    dim3 grid(xcd_grid(B * HK * ((NS + CPW - 1) / CPW)));
    hipLaunchKernelGGL(xattn_bwd_dkv_kernel<float>, grid, dim3(64 * kDkvWavesPerChapter * CPW), 0, stream, (const float*)q,
                       (const float*)dout, (const float*)k_tiles,
                       (const float*)v_tiles, slot_u, omega, lse, delta, (int)B, (int)L, Lp, H, HK, NS, su, sh, st, sl2,
                       scale, (float*)dkv_edge, domega_part);
  } else {
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dkv: dtype %d", dtype);
  }
  return check_launch("xattn_bwd_dkv_kernel");
}

int moc_dkv_reduce(int dtype, const void* dkv_edge, const int32_t* n_uniq, const int32_t* csr_off,
                   const int32_t* csr_edge, int64_t max_u, int64_t row_elems, void* dkv, hipStream_t stream) {
  MOC_REQUIRE(dkv_edge && n_uniq && csr_off && csr_edge && dkv, MOC_ERR_ARG, "moc_dkv_reduce: null pointer");
  MOC_REQUIRE(row_elems > 0 && row_elems % 8 == 0, MOC_ERR_ARG, "moc_dkv_reduce: row_elems %lld", (long long)row_elems);
  if (max_u == 0) return MOC_OK;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(dkv_reduce_kernel<bf16>, dim3((unsigned)max_u, kRedSplit), dim3(256), 0, stream, (const bf16*)dkv_edge,
                       n_uniq, csr_off, csr_edge, row_elems, (bf16*)dkv);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(dkv_reduce_kernel<float>, dim3((unsigned)max_u, kRedSplit), dim3(256), 0, stream, (const float*)dkv_edge,
                       n_uniq, csr_off, csr_edge, row_elems, (float*)dkv);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_dkv_reduce: dtype %d", dtype);
  return check_launch("dkv_reduce_kernel");
}

int moc_gather_rows(int dtype, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                    const int32_t* n_uniq, int64_t max_u, const float* row_mean, const float* row_rstd, void* out,
                    hipStream_t stream) {
  MOC_REQUIRE(bank && uniq && n_uniq && out, MOC_ERR_ARG, "moc_gather_rows: null pointer");
  MOC_REQUIRE(d % 8 == 0, MOC_ERR_UNSUPPORTED, "moc_gather_rows: d=%lld must be a multiple of 8", (long long)d);
  const int64_t rows = max_u * T;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + 3) / 4));
#define GR(TT, BT)                                                                                                     \
  hipLaunchKernelGGL((gather_rows_kernel<TT, BT>), grid, dim3(256), 0, stream, (const BT*)bank, d, T, uniq, n_uniq,   \
                     rows, row_mean, row_rstd, (TT*)out)
  if (dtype == MOC_BF16 && bank_dtype == MOC_BF16) GR(bf16, bf16);
  else if (dtype == MOC_BF16 && bank_dtype == MOC_F32) GR(bf16, float);
  else if (dtype == MOC_F32 && bank_dtype == MOC_F32) GR(float, float);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_gather_rows: dtype %d bank dtype %d", dtype, bank_dtype);
#undef GR
  return check_launch("gather_rows_kernel");
}

int moc_bank_scatter(int dx_dtype, const void* dX, const void* bank, int bank_dtype, int64_t d, int T,
                     const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                     const int32_t* csr_edge, const float* row_mean, const float* row_rstd, int norm,
                     void* grad_bank, hipStream_t stream) {
  MOC_REQUIRE(dX && bank && uniq && n_uniq && grad_bank, MOC_ERR_ARG, "moc_bank_scatter: null pointer");
  MOC_REQUIRE((csr_off == nullptr) == (csr_edge == nullptr), MOC_ERR_ARG,
              "moc_bank_scatter: csr_off / csr_edge must be both set or both null");
  MOC_REQUIRE(d % 8 == 0, MOC_ERR_UNSUPPORTED, "moc_bank_scatter: d=%lld must be a multiple of 8", (long long)d);
  MOC_REQUIRE((norm == MOC_NORM_NONE) == (row_rstd == nullptr), MOC_ERR_ARG, "moc_bank_scatter: norm/stats mismatch");
  const int64_t rows = max_u * T;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + 3) / 4));
  const int ln = norm == MOC_NORM_LAYERNORM;
#define BS(TX, BT)                                                                                                     \
  hipLaunchKernelGGL((bank_scatter_kernel<TX, BT, BT>), grid, dim3(256), 0, stream, (const TX*)dX, (const BT*)bank, d, \
                     T, uniq, n_uniq, rows, csr_off, csr_edge, row_mean, row_rstd, ln, nullptr, (BT*)grad_bank)
  if (dx_dtype == MOC_BF16 && bank_dtype == MOC_BF16) BS(bf16, bf16);
  else if (dx_dtype == MOC_BF16 && bank_dtype == MOC_F32) BS(bf16, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_F32) BS(float, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_BF16) BS(float, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_bank_scatter: dtypes %d/%d", dx_dtype, bank_dtype);
#undef BS
  return check_launch("bank_scatter_kernel");
}

int moc_fill_zero(void* dst, int64_t bytes, int workgroups, hipStream_t stream) {
  MOC_REQUIRE(dst || bytes == 0, MOC_ERR_ARG, "moc_fill_zero: null pointer");
  MOC_REQUIRE(bytes >= 0 && bytes % 16 == 0 && ((uintptr_t)dst & 15) == 0, MOC_ERR_ARG,
              "moc_fill_zero: bytes=%lld and the address must be multiples of 16", (long long)bytes);
  MOC_REQUIRE(workgroups > 0 && workgroups <= 65536, MOC_ERR_ARG, "moc_fill_zero: workgroups=%d", workgroups);
  if (bytes == 0) return MOC_OK;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)workgroups), dim3(64), 0, stream, (V16*)dst, bytes / 16);
  return check_launch("fill_zero_kernel");
}

int moc_bank_grad_accumulate(int dx_dtype, const void* dX, const void* bank, int bank_dtype, int64_t d, int T,
                             const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                             const int32_t* csr_edge, const float* row_mean, const float* row_rstd, int norm,
                             int epoch, int32_t* chap_epoch, int32_t* fresh, float* grad_acc, hipStream_t stream) {
  MOC_REQUIRE(dX && bank && uniq && n_uniq && chap_epoch && fresh && grad_acc, MOC_ERR_ARG,
              "moc_bank_grad_accumulate: null pointer");
  MOC_REQUIRE((csr_off == nullptr) == (csr_edge == nullptr), MOC_ERR_ARG,
              "moc_bank_grad_accumulate: csr_off / csr_edge must be both set or both null");
  MOC_REQUIRE(d % 8 == 0, MOC_ERR_UNSUPPORTED, "moc_bank_grad_accumulate: d=%lld must be a multiple of 8",
              (long long)d);
  MOC_REQUIRE((norm == MOC_NORM_NONE) == (row_rstd == nullptr), MOC_ERR_ARG,
              "moc_bank_grad_accumulate: norm/stats mismatch");
  if (max_u == 0) return MOC_OK;
  hipLaunchKernelGGL(bank_grad_mark_kernel, dim3((unsigned)((max_u + 255) / 256)), dim3(256), 0, stream, uniq, n_uniq,
                     max_u, epoch, chap_epoch, fresh);
  int rc = check_launch("bank_grad_mark_kernel");
  if (rc) return rc;
  const int64_t rows = max_u * T;
  dim3 grid((unsigned)((rows + 3) / 4));
  const int ln = norm == MOC_NORM_LAYERNORM;
#define BA(TX, BT)                                                                                                     \
  hipLaunchKernelGGL((bank_scatter_kernel<TX, BT, float>), grid, dim3(256), 0, stream, (const TX*)dX, (const BT*)bank, \
                     d, T, uniq, n_uniq, rows, csr_off, csr_edge, row_mean, row_rstd, ln, fresh, grad_acc)
  if (dx_dtype == MOC_BF16 && bank_dtype == MOC_BF16) BA(bf16, bf16);
  else if (dx_dtype == MOC_BF16 && bank_dtype == MOC_F32) BA(bf16, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_F32) BA(float, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_BF16) BA(float, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_bank_grad_accumulate: dtypes %d/%d", dx_dtype, bank_dtype);
#undef BA
  return check_launch("bank_scatter_kernel");
}

}  // extern "C"
