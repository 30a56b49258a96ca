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

// delta[b, h, i] = sum_d dO[b, i, h, d] * O[b, i, h, d]; 16 lanes per row.
template <typename T>
__global__ __launch_bounds__(256) void xattn_bwd_prep_kernel(const T* __restrict__ out, const T* __restrict__ dout,
                                                             int64_t rows, int L, int H, float* __restrict__ delta) {
  const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float acc = 0.f;
  if (r < rows) {
    const T* o = out + r * kBDh + 4 * sub;
    const T* d = dout + r * kBDh + 4 * sub;
#pragma unroll
    for (int x = 0; x < 4; ++x) acc += to_f(o[x]) * to_f(d[x]);
  }
#pragma unroll
  for (int s = 8; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 16);
  if (r < rows && sub == 0) {
    const int64_t h = r % H, bi = r / H;
    const int64_t i = bi % L, b = bi / L;
    delta[(b * H + h) * L + i] = acc;
  }
}

// dq: one workgroup = 128 queries of one (sequence, head), loop over its slots.
template <typename T>
__global__ __launch_bounds__(kBThreads) void xattn_bwd_dq_kernel(
    const T* __restrict__ q, const T* __restrict__ ktiles, const T* __restrict__ vtiles,
    const int32_t* __restrict__ slot_u, const float* __restrict__ omega, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int L, int H, int HK, int NS, float scale_log2,
    float scale, T* __restrict__ dq) {
  typedef typename Frag<T>::type F8;
  using Tile = SwzTile<T, 64>;
  constexpr int TB = kBT * kBDh * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) char sK[TB];
  __shared__ __attribute__((aligned(16))) char sKt[TB];
  __shared__ __attribute__((aligned(16))) char sV[TB];

  const int b = blockIdx.z, h = blockIdx.y;
  const int hk = h / (H / HK);
  const int q0 = blockIdx.x * 128;
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
    lse2[qb] = ok ? lse[((size_t)b * H + h) * L + qi] : INFINITY;
    dl[qb] = ok ? delta[((size_t)b * H + h) * L + qi] : 0.f;
  }
  f32x4 acc[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* su = slot_u + (size_t)b * NS;
  const float* om = omega + (size_t)b * NS;
  TileIO<T, kBThreads> kio, vio;
  auto tile_ptr = [&](const T* base, int u) { return base + ((size_t)u * HK + hk) * (kBT * kBDh); };
  int u_cur = su[0];
  if (u_cur >= 0) {
    kio.load(tile_ptr(ktiles, u_cur), tid);
    vio.load(tile_ptr(vtiles, u_cur), tid);
  }
  for (int s = 0; s < NS; ++s) {
    if (u_cur >= 0) {
      kio.store(sK, tid);
      kio.store_t(sKt, tid);
      vio.store(sV, tid);
    }
    __syncthreads();
    const int u_next = (s + 1 < NS) ? su[s + 1] : -1;
    if (u_next >= 0) {
      kio.load(tile_ptr(ktiles, u_next), tid);
      vio.load(tile_ptr(vtiles, u_next), tid);
    }
    if (u_cur >= 0) {
      const float w = om[s];
      const float c = w * scale_log2;
      const float dsc = w * scale;
      f32x4 st[4][2], dp[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          F8 ak = Tile::frag(sK, 16 * kb + c16, 32 * ks + 8 * g);
          F8 av = Tile::frag(sV, 16 * kb + c16, 32 * ks + 8 * g);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            mma(st[kb][qb], ak, qf[qb][ks]);
            mma(dp[kb][qb], av, dof[qb][ks]);
          }
        }
      }
      F8 dsf[2][2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p = exp2f(st[kb][qb][e] * c - lse2[qb]);
            const float ds = p * (w * dp[kb][qb][e] - dl[qb]) * dsc;
            const int ks2 = kb >> 1, half = kb & 1;
            dsf[qb][ks2][4 * half + e] = from_f<T>(ds);
          }
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          F8 bk = Tile::frag44(sKt, 16 * db + c16, 32 * ks2 + 4 * g, 32 * ks2 + 16 + 4 * g);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) mma(acc[qb][db], dsf[qb][ks2], bk);
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

// dk/dv: one workgroup per (distinct chapter u, kv head hk); walks the edges of
// u in csr order and, for each, the G query heads of hk and all L queries of
// the edge's sequence in steps of 128 (4 waves x 32 queries).  K and V of the
// chapter stay in registers; Q^T and dO^T of the step are staged in LDS.
template <typename T>
__global__ __launch_bounds__(kBThreads, 1) void xattn_bwd_dkv_kernel(
    const T* __restrict__ q, const T* __restrict__ ktiles, const T* __restrict__ vtiles,
    const float* __restrict__ omega, const T* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, const int32_t* __restrict__ n_uniq, const int32_t* __restrict__ csr_off,
    const int32_t* __restrict__ csr_edge, int L, int H, int HK, int NS, float scale_log2, float scale,
    T* __restrict__ dkv, float* __restrict__ domega_part) {
  typedef typename Frag<T>::type F8;
  constexpr int QS = 128;
  using TileQ = SwzTile<T, QS>;             // [64 dims][128 queries]
  constexpr int STAGE = kBDh * QS * (int)sizeof(T);
  constexpr int SMEM = 2 * STAGE > 32768 ? 2 * STAGE : 32768;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  __shared__ float red[kBThreads / 64];
  char* sQt = smem;
  char* sDt = smem + STAGE;

  const int u = blockIdx.x, hk = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int KV = HK * kBDh;
  const size_t row_stride = 2 * (size_t)KV;
  if (u >= n_uniq[0]) {
    // rows of unused plan slots are zero so that GEMMs over all slots stay exact
    for (int i = tid; i < kBT * kBDh; i += kBThreads) {
      const int key = i / kBDh, dim = i % kBDh;
      T* rowp = dkv + ((size_t)u * kBT + key) * row_stride;
      rowp[hk * kBDh + dim] = from_f<T>(0.f);
      rowp[KV + hk * kBDh + dim] = from_f<T>(0.f);
    }
    return;
  }
  const int G = H / HK;

  const T* Kt = ktiles + ((size_t)u * HK + hk) * (kBT * kBDh);
  const T* Vt = vtiles + ((size_t)u * HK + hk) * (kBT * kBDh);
  F8 kf[4][2], vf[4][2];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      kf[kb][ks] = Load8<T, T>::run(Kt + (16 * kb + c16) * kBDh + 32 * ks + 8 * g);
      vf[kb][ks] = Load8<T, T>::run(Vt + (16 * kb + c16) * kBDh + 32 * ks + 8 * g);
    }
  f32x4 dk[4][4], dv[4][4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      dk[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      dv[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int CPR = kBDh / EPC;
  constexpr int NCH = (QS * CPR) / kBThreads;  // chunks of each of Q and dO per thread per step

  const int p0 = csr_off[u], p1 = csr_off[u + 1];
  for (int p = p0; p < p1; ++p) {
    const int e = csr_edge[p];
    const int b = e / NS;
    const float w = omega[e];
    const float c = w * scale_log2;
    const float dsc = w * scale;
    for (int hq = hk * G; hq < hk * G + G; ++hq) {
      float dwp = 0.f;
      const size_t lrow = ((size_t)b * H + hq) * L;
      for (int q0 = 0; q0 < L; q0 += QS) {
        // stage Q^T and dO^T (transposed) for queries q0 .. q0+127
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int ch = tid + kBThreads * i;
          const int qq = ch / CPR, d0 = (ch % CPR) * EPC;
          const int qi = q0 + qq;
          V16 vq, vd;
          if (qi < L) {
            const size_t off = ((size_t)(b * (size_t)L + qi) * H + hq) * kBDh + d0;
            vq = ld16(q + off);
            vd = ld16(dout + off);
          } else {
            vq = V16{{0u, 0u, 0u, 0u}};
            vd = vq;
          }
          const T* tq = reinterpret_cast<const T*>(&vq);
          const T* td = reinterpret_cast<const T*>(&vd);
#pragma unroll
          for (int x = 0; x < EPC; ++x) {
            *reinterpret_cast<T*>(sQt + TileQ::off(d0 + x, qq)) = tq[x];
            *reinterpret_cast<T*>(sDt + TileQ::off(d0 + x, qq)) = td[x];
          }
        }
        // A-operand fragments (row = query) straight from global
        F8 qa[2][2], da[2][2];
        float l2[2][4], dl[2][4];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const int qi = q0 + 32 * wave + 16 * qb + c16;
          const bool ok = qi < L;
          const size_t off = ((size_t)(b * (size_t)L + qi) * H + hq) * kBDh;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            qa[qb][ks] = ok ? Load8<T, T>::run(q + off + 32 * ks + 8 * g) : zero_frag<T>();
            da[qb][ks] = ok ? Load8<T, T>::run(dout + off + 32 * ks + 8 * g) : zero_frag<T>();
          }
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const int qr = q0 + 32 * wave + 16 * qb + 4 * g + x;
            l2[qb][x] = qr < L ? lse[lrow + qr] : INFINITY;
            dl[qb][x] = qr < L ? delta[lrow + qr] : 0.f;
          }
        }
        // S = Q K^T and dPu = dO V^T: rows = queries 4g+x of block qb, column = key 16kb + c16
        f32x4 sc[2][4], dp[2][4];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            sc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
            dp[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
              mma(sc[qb][kb], qa[qb][ks], kf[kb][ks]);
              mma(dp[qb][kb], da[qb][ks], vf[kb][ks]);
            }
        // P^T (scaled by omega) and dS^T (scaled by omega*scale) as A operands: row = key
        F8 pa[4], sa[4];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int x = 0; x < 4; ++x) {
              const float sraw = sc[qb][kb][x];
              const float pr = exp2f(sraw * c - l2[qb][x]);
              const float dpu = dp[qb][kb][x];
              const float ds = pr * (w * dpu - dl[qb][x]);
              dwp += ds * sraw * scale + pr * dpu;
              pa[kb][4 * qb + x] = from_f<T>(pr * w);
              sa[kb][4 * qb + x] = from_f<T>(ds * dsc);
            }
        __syncthreads();  // staged Q^T / dO^T visible
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          F8 bq = TileQ::frag44(sQt, 16 * db + c16, 32 * wave + 4 * g, 32 * wave + 16 + 4 * g);
          F8 bd = TileQ::frag44(sDt, 16 * db + c16, 32 * wave + 4 * g, 32 * wave + 16 + 4 * g);
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            mma(dv[kb][db], pa[kb], bd);
            mma(dk[kb][db], sa[kb], bq);
          }
        }
        __syncthreads();  // before the next step overwrites the stage
      }
      // domega partial of (edge, query head)
      dwp = wave_sum(dwp);
      if (lane == 0) red[wave] = dwp;
      __syncthreads();
      if (tid == 0) domega_part[(size_t)e * H + hq] = red[0] + red[1] + red[2] + red[3];
      __syncthreads();
    }
  }

  // Cross-wave reduction of dk, dv (4 partial 64x64 fp32 tiles each) through LDS.
  float* buf = reinterpret_cast<float*>(smem);  // holds 2 tiles (32 KB)
  T* rows = dkv + (size_t)u * kBT * row_stride;
  auto reduce_store = [&](f32x4 (&acc)[4][4], int col0) {
    // round 1: waves 2,3 publish; waves 0,1 add
    if (wave >= 2) {
      float* t = buf + (wave - 2) * 4096;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int x = 0; x < 4; ++x) t[(16 * kb + 4 * g + x) * 64 + 16 * db + c16] = acc[kb][db][x];
    }
    __syncthreads();
    if (wave < 2) {
      const float* t = buf + wave * 4096;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int x = 0; x < 4; ++x) acc[kb][db][x] += t[(16 * kb + 4 * g + x) * 64 + 16 * db + c16];
    }
    __syncthreads();
    // round 2: wave 1 publishes, wave 0 adds and writes the rows
    if (wave == 1) {
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
          for (int x = 0; x < 4; ++x) {
            const int key = 16 * kb + 4 * g + x, dim = 16 * db + c16;
            rows[(size_t)key * row_stride + col0 + dim] = from_f<T>(acc[kb][db][x] + buf[key * 64 + dim]);
          }
    }
    __syncthreads();
  };
  reduce_store(dk, hk * kBDh);
  reduce_store(dv, KV + hk * kBDh);
}

// X[r, :] = norm(bank[uniq[r / T] * T + r % T, :]) in the compute dtype; rows of
// unused plan slots (r >= n_uniq * T) are zero.
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
  if (r >= valid) {
    for (int64_t j = lane; j < d; j += 64) o[j] = from_f<T>(0.f);
    return;
  }
  const TB* x = bank + ((int64_t)uniq[r / Tc] * Tc + r % Tc) * d;
  const float mu = rstd ? mean[r] : 0.f, rs = rstd ? rstd[r] : 1.f;
  for (int64_t j = lane; j < d; j += 64) o[j] = from_f<T>((to_f(x[j]) - mu) * rs);
}

// grad_bank[src(r), :] = norm_bwd(dX[r, :]) for r < n_uniq * T.  Distinct
// chapters own distinct bank rows, so plain stores suffice (grad_bank must be
// zero-initialised by the caller for rows that are not selected).
template <typename TX, typename TB, typename TG>
__global__ __launch_bounds__(256) void bank_scatter_kernel(const TX* __restrict__ dX, const TB* __restrict__ bank,
                                                           int64_t d, int Tc, const int32_t* __restrict__ uniq,
                                                           const int32_t* __restrict__ n_uniq, int64_t rows,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd, int layernorm,
                                                           TG* __restrict__ grad) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows || r >= (int64_t)n_uniq[0] * Tc) return;
  const int64_t src = (int64_t)uniq[r / Tc] * Tc + r % Tc;
  const TX* g = dX + r * d;
  TG* o = grad + src * d;
  if (!rstd) {
    for (int64_t j = lane; j < d; j += 64) o[j] = (TG)to_f(g[j]);
    return;
  }
  const TB* x = bank + src * d;
  const float mu = mean[r], rs = rstd[r];
  float sg = 0.f, sgx = 0.f;
  for (int64_t j = lane; j < d; j += 64) {
    const float gv = to_f(g[j]);
    const float xh = (to_f(x[j]) - mu) * rs;
    sg += gv;
    sgx += gv * xh;
  }
  sg = wave_sum(sg) / (float)d;
  sgx = wave_sum(sgx) / (float)d;
  for (int64_t j = lane; j < d; j += 64) {
    const float gv = to_f(g[j]);
    const float xh = (to_f(x[j]) - mu) * rs;
    o[j] = (TG)(rs * (gv - (layernorm ? sg : 0.f) - xh * sgx));
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_xattn_bwd_prep(int dtype, const void* out, const void* dout, int64_t B, int64_t L, int H, int Dh,
                       float* delta, hipStream_t stream) {
  MOC_REQUIRE(out && dout && delta, MOC_ERR_ARG, "moc_xattn_bwd_prep: null pointer");
  MOC_REQUIRE(Dh == kBDh, MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_prep: head_dim %d (needs 64)", Dh);
  const int64_t rows = B * L * H;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + 15) / 16));
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_bwd_prep_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)out, (const bf16*)dout,
                       rows, (int)L, H, delta);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_bwd_prep_kernel<float>, grid, dim3(256), 0, stream, (const float*)out, (const float*)dout,
                       rows, (int)L, H, delta);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_prep: dtype %d", dtype);
  return check_launch("xattn_bwd_prep_kernel");
}

int moc_xattn_bwd_dq(int dtype, const void* q, const void* k_tiles, const void* v_tiles, const int32_t* slot_u,
                     const float* omega, const void* dout, const float* lse, const float* delta, int64_t B, int64_t L,
                     int H, int HK, int Dh, int T, int NS, float scale, void* dq, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && slot_u && omega && dout && lse && delta && dq, MOC_ERR_ARG,
              "moc_xattn_bwd_dq: null pointer");
  MOC_REQUIRE(Dh == kBDh && T == kBT, MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dq: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0, MOC_ERR_ARG, "moc_xattn_bwd_dq: bad shape");
  if (B == 0 || L == 0) return MOC_OK;
  dim3 grid((unsigned)((L + 127) / 128), (unsigned)H, (unsigned)B);
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_bwd_dq_kernel<bf16>, grid, dim3(kBThreads), 0, stream, (const bf16*)q, (const bf16*)k_tiles,
                       (const bf16*)v_tiles, slot_u, omega, (const bf16*)dout, lse, delta, (int)L, H, HK, NS, sl2, scale,
                       (bf16*)dq);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_bwd_dq_kernel<float>, grid, dim3(kBThreads), 0, stream, (const float*)q,
                       (const float*)k_tiles, (const float*)v_tiles, slot_u, omega, (const float*)dout, lse, delta,
                       (int)L, H, HK, NS, sl2, scale, (float*)dq);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dq: dtype %d", dtype);
  return check_launch("xattn_bwd_dq_kernel");
}

int moc_xattn_bwd_dkv(int dtype, const void* q, const void* k_tiles, const void* v_tiles, const float* omega,
                      const void* dout, const float* lse, const float* delta, const int32_t* n_uniq,
                      const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u, int64_t B, int64_t L, int H,
                      int HK, int Dh, int T, int NS, float scale, void* dkv, float* domega_part,
                      hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && omega && dout && lse && delta && n_uniq && csr_off && csr_edge && dkv &&
                  domega_part,
              MOC_ERR_ARG, "moc_xattn_bwd_dkv: null pointer");
  MOC_REQUIRE(Dh == kBDh && T == kBT, MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dkv: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0 && max_u >= 0, MOC_ERR_ARG, "moc_xattn_bwd_dkv: bad shape");
  if (max_u == 0) return MOC_OK;
  dim3 grid((unsigned)max_u, (unsigned)HK);
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(xattn_bwd_dkv_kernel<bf16>, grid, dim3(kBThreads), 0, stream, (const bf16*)q,
                       (const bf16*)k_tiles, (const bf16*)v_tiles, omega, (const bf16*)dout, lse, delta, n_uniq, csr_off,
                       csr_edge, (int)L, H, HK, NS, sl2, scale, (bf16*)dkv, domega_part);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(xattn_bwd_dkv_kernel<float>, grid, dim3(kBThreads), 0, stream, (const float*)q,
                       (const float*)k_tiles, (const float*)v_tiles, omega, (const float*)dout, lse, delta, n_uniq,
                       csr_off, csr_edge, (int)L, H, HK, NS, sl2, scale, (float*)dkv, domega_part);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_xattn_bwd_dkv: dtype %d", dtype);
  return check_launch("xattn_bwd_dkv_kernel");
}

int moc_gather_rows(int dtype, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                    const int32_t* n_uniq, int64_t max_u, const float* row_mean, const float* row_rstd, void* out,
                    hipStream_t stream) {
  MOC_REQUIRE(bank && uniq && n_uniq && out, MOC_ERR_ARG, "moc_gather_rows: null pointer");
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
                     const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const float* row_mean,
                     const float* row_rstd, int norm, void* grad_bank, hipStream_t stream) {
  MOC_REQUIRE(dX && bank && uniq && n_uniq && grad_bank, MOC_ERR_ARG, "moc_bank_scatter: null pointer");
  MOC_REQUIRE((norm == MOC_NORM_NONE) == (row_rstd == nullptr), MOC_ERR_ARG, "moc_bank_scatter: norm/stats mismatch");
  const int64_t rows = max_u * T;
  if (rows == 0) return MOC_OK;
  dim3 grid((unsigned)((rows + 3) / 4));
  const int ln = norm == MOC_NORM_LAYERNORM;
#define BS(TX, BT)                                                                                                     \
  hipLaunchKernelGGL((bank_scatter_kernel<TX, BT, BT>), grid, dim3(256), 0, stream, (const TX*)dX, (const BT*)bank, d, \
                     T, uniq, n_uniq, rows, row_mean, row_rstd, ln, (BT*)grad_bank)
  if (dx_dtype == MOC_BF16 && bank_dtype == MOC_BF16) BS(bf16, bf16);
  else if (dx_dtype == MOC_BF16 && bank_dtype == MOC_F32) BS(bf16, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_F32) BS(float, float);
  else if (dx_dtype == MOC_F32 && bank_dtype == MOC_BF16) BS(float, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_bank_scatter: dtypes %d/%d", dx_dtype, bank_dtype);
#undef BS
  return check_launch("bank_scatter_kernel");
}

}  // extern "C"
