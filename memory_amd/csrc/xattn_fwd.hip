// Sequence-routed memory cross-attention, forward ("joint" combine).
//
// For sequence b, query i, query head h (kv head hk = h / (H / HK)) and the
// NS selected chapters c with router weights omega[b, c]:
//   s_ij  = omega_c * scale * q_i . k_j           (j ranges over chapter c's T keys)
//   o_i   = sum_j softmax_j(s_ij) * omega_c * v_j
// which is exactly MemoryCrossAttention over the omega-weighted gathered rows
// (memory_transformer/model.py:689-692 then memory_attention.py:458-478 /
// :269-318): (omega x) W^T = omega (x W^T), so the key and the value of every
// row of chapter c carry the factor omega_c.  k_j / v_j are read as (chapter, kv head)
// blocks of 64 rows through strides (projection rows [u*64 + t][K | V] on the training
// path, kv_project.hip's chapter-head tiles for the decode cache); slot_u[b, c] says which
// de-duplicated chapter holds slot c of sequence b (negative = skip the slot).
//
// Work decomposition (Dh = T = 64): one workgroup = 128 queries of one
// (sequence, head); 4 waves x 32 queries.  Every chapter is one 64-key tile,
// so omega is a scalar per tile and folds into the exp2 argument.  Each wave
// computes S^T = K Q^T (lane = one query, 16 keys), keeps the running max,
// accumulates O^T = V^T P^T, whose accumulator layout is again "lane = one
// query", so the online-softmax rescale needs no data movement, and takes the
// row sums from an MFMA of an all-ones operand with the same P^T fragments.
// K and V blocks (both [key][dim]) are double-buffered in
// LDS; the V^T operand is read from the V tile with the transposing LDS read, whose lane
// order is the key order of the P~^T fragments.
#include "moc_common.h"

namespace moc {

constexpr int kFwdThreads = 256;
constexpr int kDh = 64;
constexpr int kTch = 64;

// Running-max policy: a row's reference max m only moves up when the chapter
// max exceeds it by more than kRescaleSlack (log2 units), so most chapters skip
// the O / l rescale; probabilities stay <= 2^kRescaleSlack, far from overflow.
constexpr float kRescaleSlack = 8.f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float max3f(float a, float b, float c) { return fmax_fast(fmax_fast(a, b), c); }
// max over the lanes {l, l^16, l^32, l^48} (the four row groups of a 16x16 accumulator column)
// with the gfx950 row-swap permutes.  v_permlane16_swap_b32 a, b swaps the odd 16-lane rows of
// a with the even rows of b (v_permlane32_swap_b32: the upper 32 lanes of a with the lower 32 of
// b); from two copies of v it leaves v's partner-row values in one of the copies.
__device__ __forceinline__ float quad_max_pl(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  float c = fmax_fast(a, b), d = c;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return fmax_fast(c, d);
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes at voff + soff
// of the buffer land at LDS address m0 + 16 l.  The wait on these loads is an explicit vmcnt(0).
typedef __attribute__((address_space(3))) void* fwd_lds_ptr_t;
__device__ __forceinline__ void fwd_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, const char* lds, uint32_t soff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(fwd_lds_ptr_t)lds;
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0) : "memory");
}

template <typename T>
__global__ __launch_bounds__(kFwdThreads) void xattn_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ ktiles, const T* __restrict__ vtiles,
    const int32_t* __restrict__ slot_u, const float* __restrict__ omega, int B, int L, int H, int HK, int NS,
    int64_t kv_span, int64_t kv_su, int kv_sh, int kv_st, float scale_log2, T* __restrict__ out, float* __restrict__ lse) {
  typedef typename Frag<T>::type F8;
  using Tile = SwzTile<T, 64>;
  constexpr int TB = kTch * kDh * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) char sK[2][TB];
  __shared__ __attribute__((aligned(16))) char sV[2][TB];

  // tiles: (sequence, head) major, 128-query block minor, so the query blocks that read
  // the same chapter tiles share one XCD's L2
  const int nqb = (L + 127) / 128;
  const int64_t t = xcd_tile((int64_t)B * H * nqb);
  if (t < 0) return;
  const int b = (int)(t / ((int64_t)H * nqb)), h = (int)((t / nqb) % H);
  const int hk = h / (H / HK);
  const int q0 = (int)(t % nqb) * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;

  // Q^T fragments (B operand): query = q0 + 32*wave + 16*qb + c16, dims 32*ks + 8*g ..
  F8 qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = q0 + 32 * wave + 16 * qb + c16;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (qi < L)
        qf[qb][ks] = Load8<T, T>::run(q + ((size_t)(b * (size_t)L + qi) * H + h) * kDh + 32 * ks + 8 * g);
      else
        qf[qb][ks] = zero_frag<T>();
    }
  }

  float m[2] = {-INFINITY, -INFINITY};
  float lsum[2] = {0.f, 0.f};  // row sums of p (in units of exp2(m)), complete per lane
  float pend_ls[2] = {0.f, 0.f}, pend_rw = 0.f;   // last chapter's row sums, not yet folded in
  // all-ones A operand: the MFMA with it sums a P~^T fragment over its 32 keys, which
  // takes the row sums off the VALU (the sums use the same rounded P~ as O)
  F8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = from_f<T>(1.f);
  f32x4 o[4][2];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* su = slot_u + (size_t)b * NS;
  const float* om = omega + (size_t)b * NS;
  TileIO<T, kFwdThreads> kio, vio;
  // block (u, hk) of K / V: element (t, dh) at u kv_su + hk kv_sh + t kv_st + dh of two buffers of
  // kv_span elements each
  const Buf kb(ktiles, (uint32_t)(kv_span * (int64_t)sizeof(T))), vb(vtiles, (uint32_t)(kv_span * (int64_t)sizeof(T)));
  auto tile_off = [&](int u) { return (uint32_t)(((size_t)u * kv_su + (size_t)hk * kv_sh) * sizeof(T)); };
  const uint32_t row_bytes = (uint32_t)(kv_st * (int)sizeof(T));
  // bf16: a slot's K and V tiles go global -> LDS by DMA (no registers held while in flight):
  // 8 instructions of 1 KB (8 rows of 128 B) per tile, wave w issuing 2w and 2w + 1; lane l fills
  // row 8 j + l / 8, physical chunk l % 8 = logical chunk (l % 8) ^ (row & 7) of Tile::off.
  // fp32: through registers.
  constexpr bool kDma = sizeof(T) == 2;
  static_assert(!kDma || (kFwdThreads == 256 && TB == 8192), "DMA staging geometry");
  const uint32_t dma_v0 = (uint32_t)((16 * wave + (lane >> 3)) * row_bytes + 16 * ((lane & 7) ^ (lane >> 3)));
  auto fetch = [&](int u, int buf) {
    if constexpr (kDma) {
      const uint32_t so = tile_off(u);
      fwd_dma16(kb.r, dma_v0, sK[buf] + 2048 * wave, so);
      fwd_dma16(kb.r, dma_v0 + 8 * row_bytes, sK[buf] + 2048 * wave + 1024, so);
      fwd_dma16(vb.r, dma_v0, sV[buf] + 2048 * wave, so);
      fwd_dma16(vb.r, dma_v0 + 8 * row_bytes, sV[buf] + 2048 * wave + 1024, so);
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
  // Q fragments must have landed before the loop on every path (also when slot 0
  // is skipped); otherwise the wait for them inside the loop can't be told apart
  // from the prefetch and becomes a full vmcnt(0) ahead of the first MFMA.
  vm_wait_all();
  __syncthreads();

  for (int s = 0; s < NS; ++s) {
    const int buf = s & 1;
    const int u_next = (s + 1 < NS) ? su[s + 1] : -1;
    // (buffer buf ^ 1 was last read in slot s - 1, which every wave has finished)
    if (u_next >= 0) fetch(u_next, buf ^ 1);
    if (u_cur >= 0) {
      const float w = om[s];
      const float c = w * scale_log2;
      const char* Ks = sK[buf];
      const char* Vs = sV[buf];
      // S^T[kb][qb]: rows = keys 16*kb + 4*g + e, column = query c16 of block qb
      f32x4 st[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          F8 a = Tile::frag(Ks, 16 * kb + c16, 32 * ks + 8 * g);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) mma(st[kb][qb], a, qf[qb][ks]);
        }
      }
      // the previous chapter's row sums (their MFMA has long completed): folded in before any
      // rescale, in units of the reference max they were taken against
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) lsum[qb] += pend_ls[qb] * pend_rw;
      pend_rw = 0.f;
      // chapter max per row (three-input max chains), lazy update of the reference max
      float cm[2];
      bool grow = false;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float mx = max3f(st[0][qb][0], st[0][qb][1], st[0][qb][2]);
        mx = max3f(mx, st[0][qb][3], st[1][qb][0]);
        mx = max3f(mx, st[1][qb][1], st[1][qb][2]);
        mx = max3f(mx, st[1][qb][3], st[2][qb][0]);
        mx = max3f(mx, st[2][qb][1], st[2][qb][2]);
        mx = max3f(mx, st[2][qb][3], st[3][qb][0]);
        mx = max3f(mx, st[3][qb][1], st[3][qb][2]);
        mx = fmax_fast(mx, st[3][qb][3]);
        cm[qb] = quad_max_pl(mx) * c;  // c >= 0 (router weights are non-negative)
        grow |= cm[qb] > m[qb] + kRescaleSlack;
      }
      if (__any(grow)) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float mn = cm[qb] > m[qb] + kRescaleSlack ? cm[qb] : m[qb];
          const float alpha = fast_exp2(m[qb] - mn);
          m[qb] = mn;
          lsum[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < 4; ++db) o[db][qb] *= alpha;
        }
      }
      F8 pf[2][2];
      if (w > kTinyOmega) {
        // p~ = w * exp2(s*c - m): w folded into the exponent; the row sum needs sum(p~) / w
        const float lw = __builtin_amdgcn_logf(w);
        const float rw = __builtin_amdgcn_rcpf(w);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float off = m[qb] - lw;
#pragma unroll
          for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              pf[qb][ks2][e] = from_f<T>(fast_exp2(st[2 * ks2][qb][e] * c - off));
              pf[qb][ks2][4 + e] = from_f<T>(fast_exp2(st[2 * ks2 + 1][qb][e] * c - off));
            }
          f32x4 ls = f32x4{0.f, 0.f, 0.f, 0.f};
          mma(ls, ones, pf[qb][0]);
          mma(ls, ones, pf[qb][1]);
          pend_ls[qb] = ls[0];   // folded in at the next chapter (no wait on this MFMA here)
        }
        pend_rw = rw;
        // O^T[db][qb] += V^T(dims 16*db + c16, keys) * P~^T
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2) {
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const F8 a = mk_frag<Tile, T>(Vs, 32 * ks2, 16 * db, lane);  // V^T, keys in MFMA key order
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) mma(o[db][qb], a, pf[qb][ks2]);
          }
        }
      } else {
        // zero (or below-floor) weight: keys and values vanish, every logit is 0 -> only the
        // denominator moves
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) lsum[qb] += 64.f * fast_exp2(-m[qb]);
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
  for (int qb = 0; qb < 2; ++qb) lsum[qb] += pend_ls[qb] * pend_rw;
  // lse rows have stride Lp = round_up(L, 128); padded entries hold +inf so
  // that the backward's exp2(s - lse) is exactly 0 there (also for a row
  // whose every slot was skipped).
  const int Lp = nqb * 128;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l = lsum[qb];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int qi = q0 + 32 * wave + 16 * qb + c16;
    if (qi < L) {
      T* op = out + ((size_t)(b * (size_t)L + qi) * H + h) * kDh;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int e = 0; e < 4; ++e) op[16 * db + 4 * g + e] = from_f<T>(o[db][qb][e] * inv);
    }
    if (g == 0) lse[((size_t)b * H + h) * Lp + qi] = (qi < L && l > 0.f) ? m[qb] + log2f(l) : INFINITY;
  }
}

// Attention weights of the forward above, materialised (MemoryCrossAttention.forward with
// return_attn_weights, memory_attention.py:437-447: softmax(q k^T * scale) over the sequence's
// selected keys, which carry omega): p_ij = exp2(omega_c scale log2(e) q_i . k_j - lse_i) with the
// forward's row log-sum-exp.  One workgroup = 64 queries x one slot of one (sequence, head), wave w
// owning queries 16 w .. 16 w + 15: S^T = K Q^T from global fragments (lane = query, 16 keys per
// lane), then 4 consecutive keys per store.  A skipped slot's keys get weight 0; a slot below the
// omega floor gets every logit 0 (its keys vanish), as in the forward.
template <typename T>
__global__ __launch_bounds__(256) void xattn_weights_kernel(
    const T* __restrict__ q, const T* __restrict__ ktiles, const int32_t* __restrict__ slot_u,
    const float* __restrict__ omega, int B, int L, int H, int HK, int NS, int64_t kv_span, int64_t kv_su, int kv_sh,
    int kv_st, float scale_log2, const float* __restrict__ lse, T* __restrict__ P) {
  typedef typename Frag<T>::type F8;
  const int nqb = (L + 63) / 64;
  const int64_t t = blockIdx.x;
  const int s = (int)(t % NS);
  const int64_t r = t / NS;
  const int qb = (int)(r % nqb);
  const int h = (int)((r / nqb) % H), b = (int)(r / ((int64_t)nqb * H));
  const int hk = h / (H / HK);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int qi = qb * 64 + 16 * wave + c16;
  const int Lp = (L + 127) / 128 * 128;
  const int u = slot_u[(size_t)b * NS + s];
  const float w = omega[(size_t)b * NS + s];
  const float lq = qi < L ? lse[((size_t)b * H + h) * Lp + qi] : 0.f;
  f32x4 st[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) st[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (u >= 0 && w > kTinyOmega) {
    F8 qf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qf[ks] = qi < L ? Load8<T, T>::run(q + ((size_t)(b * (size_t)L + qi) * H + h) * kDh + 32 * ks + 8 * g)
                      : zero_frag<T>();
    // K block (u, hk) through a bounded buffer resource (reads past kv_span return zero)
    const Buf kbuf(ktiles, (uint32_t)(kv_span * (int64_t)sizeof(T)));
    const uint32_t soff = (uint32_t)(((size_t)u * kv_su + (size_t)hk * kv_sh) * sizeof(T));
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t voff = (uint32_t)(((16 * kb + c16) * kv_st + 32 * ks + 8 * g) * (int)sizeof(T));
        F8 a;
        if constexpr (sizeof(T) == 2) {
          a = __builtin_bit_cast(F8, kbuf.load16(voff, soff));
        } else {
          const V16 lo = kbuf.load16(voff, soff), hi = kbuf.load16(voff + 16, soff);
          a = F8{__uint_as_float(lo.w[0]), __uint_as_float(lo.w[1]), __uint_as_float(lo.w[2]), __uint_as_float(lo.w[3]),
                 __uint_as_float(hi.w[0]), __uint_as_float(hi.w[1]), __uint_as_float(hi.w[2]), __uint_as_float(hi.w[3])};
        }
        mma(st[kb], a, qf[ks]);
      }
  }
  if (qi >= L) return;
  const float c = w * scale_log2;
  T* row = P + (((size_t)b * H + h) * L + qi) * ((size_t)NS * kTch) + (size_t)s * kTch;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    T v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = from_f<T>(u < 0 ? 0.f : fast_exp2(st[kb][e] * c - lq));
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<bf16x4*>(row + 16 * kb + 4 * g) = bf16x4{v[0], v[1], v[2], v[3]};
    } else {
      *reinterpret_cast<f32x4*>(row + 16 * kb + 4 * g) = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_xattn_fwd(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span, int64_t su,
                  int sh, int st, const int32_t* slot_u, const float* omega, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                  int NS, float scale, void* out, float* lse, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && slot_u && omega && out && lse, MOC_ERR_ARG, "moc_xattn_fwd: null pointer");
  MOC_REQUIRE(Dh == kDh && T == kTch, MOC_ERR_UNSUPPORTED, "moc_xattn_fwd: needs head_dim 64 and 64 tokens per chapter (got %d, %d)", Dh, T);
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0, MOC_ERR_ARG, "moc_xattn_fwd: H=%d HK=%d", H, HK);
  MOC_REQUIRE(NS > 0 && B >= 0 && L >= 0, MOC_ERR_ARG, "moc_xattn_fwd: bad shape");
  MOC_REQUIRE(B < 65536 && H < 65536, MOC_ERR_UNSUPPORTED, "moc_xattn_fwd: grid too large");
  if (int rc = check_kv_layout("moc_xattn_fwd", dtype, kv_span, su, sh, st)) return rc;
  if (B == 0 || L == 0) return MOC_OK;
  MOC_REQUIRE(B * H * ((L + 127) / 128) < ((int64_t)1 << 31), MOC_ERR_UNSUPPORTED, "moc_xattn_fwd: grid too large");
  dim3 grid(xcd_grid(B * H * ((L + 127) / 128)));
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_fwd_kernel<bf16>, grid, dim3(kFwdThreads), 0, stream, (const bf16*)q, (const bf16*)k_tiles,
                       (const bf16*)v_tiles, slot_u, omega, (int)B, (int)L, H, HK, NS, kv_span, su, sh, st, sl2, (bf16*)out, lse);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_fwd_kernel<float>, grid, dim3(kFwdThreads), 0, stream, (const float*)q,
                       (const float*)k_tiles, (const float*)v_tiles, slot_u, omega, (int)B, (int)L, H, HK, NS, kv_span, su, sh, st,
                       sl2, (float*)out, lse);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_fwd: dtype %d", dtype);
  return check_launch("xattn_fwd_kernel");
}

int moc_xattn_weights(int dtype, const void* q, const void* k_tiles, int64_t kv_span, int64_t su, int sh, int st,
                      const int32_t* slot_u, const float* omega, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                      int NS, float scale, const float* lse, void* weights, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && slot_u && omega && lse && weights, MOC_ERR_ARG, "moc_xattn_weights: null pointer");
  MOC_REQUIRE(Dh == kDh && T == kTch, MOC_ERR_UNSUPPORTED,
              "moc_xattn_weights: needs head_dim 64 and 64 tokens per chapter (got %d, %d)", Dh, T);
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0 && B >= 0 && L >= 0, MOC_ERR_ARG, "moc_xattn_weights: bad shape");
  if (int rc = check_kv_layout("moc_xattn_weights", dtype, kv_span, su, sh, st)) return rc;
  MOC_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k_tiles & 15) == 0 && ((uintptr_t)weights & 15) == 0,
              MOC_ERR_ARG, "moc_xattn_weights: q, K and the weights must be 16-byte aligned");
  if (B == 0 || L == 0) return MOC_OK;
  const int64_t blocks = B * H * ((L + 63) / 64) * NS;
  MOC_REQUIRE(blocks < ((int64_t)1 << 31), MOC_ERR_UNSUPPORTED, "moc_xattn_weights: grid too large");
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_weights_kernel<bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, (const bf16*)q,
                       (const bf16*)k_tiles, slot_u, omega, (int)B, (int)L, H, HK, NS, kv_span, su, sh, st, sl2, lse,
                       (bf16*)weights);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_weights_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, stream, (const float*)q,
                       (const float*)k_tiles, slot_u, omega, (int)B, (int)L, H, HK, NS, kv_span, su, sh, st, sl2, lse,
                       (float*)weights);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_weights: dtype %d", dtype);
  return check_launch("xattn_weights_kernel");
}

}  // extern "C"
