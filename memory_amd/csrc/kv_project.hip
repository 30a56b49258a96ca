// Chapter gather + K/V projection as one MFMA GEMM.
//
//   rows r = u * T + j of the de-duplicated chapter list (u < n_uniq, j < T)
//   X[r, :]  = norm(bank[uniq[u] * T + j, :])        (gather + optional row norm)
//   Y[r, n]  = sum_k X[r, k] * Wkv[n, k]              Wkv = [Wk; Wv], (2*HK*Dh, d)
//
// The output is written as "chapter-head tiles": K[u][hk][j][dh] and
// V[u][hk][j][dh], i.e. every (chapter, kv head) pair is one contiguous T x Dh
// block that the attention kernels stream straight into LDS.
//
// Reference: the gather is ChapteredMemoryBank.get_chapters_batched
// (memory_transformer/memory_bank.py:263-293), the optional normalisation is
// MemoryTransformer._normalize_shared_routed_memory_vectors
// (memory_transformer/model.py:393-432, applied per row, so shared and routed
// slices need no separate pass), and the projections are k_proj / v_proj of
// MemoryCrossAttention._compute_qkv (memory_transformer/memory_attention.py:241-243).
// The router weight omega (model.py:689-692) is NOT applied here: since
// (omega * x) W^T = omega * (x W^T), it is applied per chapter inside attention,
// which lets one projected chapter serve every sequence that selected it.
#include "moc_common.h"

#include <type_traits>

namespace moc {

// Per-row statistics for the normalisation prologue: mean (layernorm only) and
// 1/sqrt(var + eps) (layernorm) or 1/sqrt(mean(x^2) + eps) (rms).
template <typename TB>
__global__ __launch_bounds__(256) void row_stats_kernel(const TB* __restrict__ bank, int64_t d, int Tc,
                                                        const int32_t* __restrict__ uniq,
                                                        const int32_t* __restrict__ n_uniq, int64_t max_u,
                                                        int norm, float eps, float* __restrict__ mean,
                                                        float* __restrict__ rstd) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t nrows = (int64_t)min((int64_t)n_uniq[0], max_u) * Tc;
  if (r >= nrows) return;
  const int64_t src = (int64_t)uniq[r / Tc] * Tc + (r % Tc);
  const TB* x = bank + src * d;
  float s = 0.f, s2 = 0.f;
  for (int64_t j = lane; j < d; j += 64) {
    float v = to_f(x[j]);
    s += v;
    s2 += v * v;
  }
  s = wave_sum(s);
  s2 = wave_sum(s2);
  if (norm == MOC_NORM_LAYERNORM) {  // biased variance, two-pass, like F.layer_norm
    const float mu = s / (float)d;
    float q = 0.f;
    for (int64_t j = lane; j < d; j += 64) {
      float v = to_f(x[j]) - mu;
      q += v * v;
    }
    q = wave_sum(q);
    if (lane == 0) { mean[r] = mu; rstd[r] = rsqrtf(q / (float)d + eps); }
  } else if (lane == 0) {
    mean[r] = 0.f;
    rstd[r] = rsqrtf(s2 / (float)d + eps);
  }
}

// EPC consecutive elements of TB as floats (EPC = 16 bytes worth of T).
template <typename T, typename TB> struct ChunkLoad;
template <> struct ChunkLoad<bf16, bf16> {
  static __device__ __forceinline__ void run(const bf16* p, float* o) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int x = 0; x < 8; ++x) o[x] = (float)v[x];
  }
};
template <> struct ChunkLoad<bf16, float> {
  static __device__ __forceinline__ void run(const float* p, float* o) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int x = 0; x < 4; ++x) { o[x] = a[x]; o[4 + x] = b[x]; }
  }
};
template <> struct ChunkLoad<float, float> {
  static __device__ __forceinline__ void run(const float* p, float* o) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int x = 0; x < 4; ++x) o[x] = a[x];
  }
};

constexpr int kGemmThreads = 256;

// 128 x 128 output tile per workgroup, 4 waves in a 2 x 2 grid of 64 x 64.
// The k-stage is 128 bytes of each row (64 bf16 / 32 fp32), double-buffered.
template <typename T, typename TB>
__global__ __launch_bounds__(kGemmThreads) void kv_project_kernel(
    const TB* __restrict__ bank, int64_t d, int Tc, const int32_t* __restrict__ uniq,
    const int32_t* __restrict__ n_uniq, int64_t max_u, const float* __restrict__ row_mean,
    const float* __restrict__ row_rstd, const T* __restrict__ wkv, int HK, int Dh, int n_mblk, int n_nblk,
    T* __restrict__ kout, T* __restrict__ vout, T* __restrict__ kout_t, T* __restrict__ vout_t) {
  constexpr int BK = 128 / (int)sizeof(T);  // elements per 128-byte row slice
  constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int KSTEPS = BK / 32;
  constexpr int TILE_BYTES = 128 * 128;
  using Tile = SwzTile<T, BK>;
  __shared__ __attribute__((aligned(16))) char lds[2][2][TILE_BYTES];

  // XCD-aware raster: workgroups are dealt round-robin to the 8 XCDs, so tile t =
  // (w % 8) * per + w / 8 gives each XCD a contiguous range of tiles, and all N blocks
  // of a row block (which share its gathered bank rows) run on one XCD's L2.
  const int w = blockIdx.x, per = (int)(gridDim.x / 8);
  const int t = (w % 8) * per + w / 8;
  if (t >= n_mblk * n_nblk) return;
  const int64_t nrows = (int64_t)min((int64_t)n_uniq[0], max_u) * Tc;
  const int64_t m0 = (int64_t)(t / n_nblk) * 128;
  if (m0 >= nrows) return;
  const int n0 = (t % n_nblk) * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 4, c16 = lane & 15;

  // Each thread moves 4 chunks of A and 4 chunks of B per stage (8 chunks per row).
  const TB* a_src[4];
  float a_mu[4], a_rs[4];
  bool a_ok[4];
  const T* b_src[4];
  int a_row[4], a_cc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + kGemmThreads * i;
    a_row[i] = q >> 3;
    a_cc[i] = q & 7;
    const int64_t r = m0 + a_row[i];
    a_ok[i] = r < nrows;
    const int64_t rr = a_ok[i] ? r : 0;
    const int64_t src = (int64_t)uniq[rr / Tc] * Tc + (rr % Tc);
    a_src[i] = bank + src * d + a_cc[i] * EPC;
    a_mu[i] = row_rstd ? row_mean[rr] : 0.f;
    a_rs[i] = row_rstd ? row_rstd[rr] : 1.f;
    b_src[i] = wkv + (int64_t)(n0 + a_row[i]) * d + a_cc[i] * EPC;
  }

  typedef typename Frag<T>::type F8;
  // Raw global data is held in registers across the MFMA loop and only
  // converted / normalised when it is written to LDS (stash), so the loads
  // of stage k+1 overlap the math of stage k.
  constexpr int NV = (EPC * (int)sizeof(TB)) / 16;  // 16-byte loads per A chunk
  V16 ra[4][NV], rb[4];
  auto fetch = [&](int kt) {
    const int64_t ko = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int x = 0; x < NV; ++x) ra[i][x] = ld16(a_src[i] + ko + x * (16 / (int)sizeof(TB)));
      rb[i] = ld16(b_src[i] + ko);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      V16 av;
      if (std::is_same<T, TB>::value && !row_rstd) {
        av = a_ok[i] ? ra[i][0] : V16{{0u, 0u, 0u, 0u}};
      } else {
        float v[EPC];
        ChunkLoad<T, TB>::run(reinterpret_cast<const TB*>(ra[i]), v);
        if (row_rstd) {
#pragma unroll
          for (int x = 0; x < EPC; ++x) v[x] = (v[x] - a_mu[i]) * a_rs[i];
        }
        if (!a_ok[i]) {
#pragma unroll
          for (int x = 0; x < EPC; ++x) v[x] = 0.f;
        }
        T tv[EPC];
#pragma unroll
        for (int x = 0; x < EPC; ++x) tv[x] = from_f<T>(v[x]);
        av = *reinterpret_cast<V16*>(tv);
      }
      st16(&lds[buf][0][Tile::off(a_row[i], a_cc[i] * EPC)], av);
      st16(&lds[buf][1][Tile::off(a_row[i], a_cc[i] * EPC)], rb[i]);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)(d / BK);
  fetch(0);
  stash(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) fetch(kt + 1);
    const char* As = lds[buf][0];
    const char* Bs = lds[buf][1];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      F8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = Tile::frag(As, wm * 64 + 16 * i + c16, ks * 32 + 8 * g);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Tile::frag(Bs, wn * 64 + 16 * j + c16, ks * 32 + 8 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) mma(acc[i][j], a[i], b[j]);
    }
    if (kt + 1 < nk) stash(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: scatter into chapter-head tiles [u][hk][t][dh]; optionally also the
  // transposed tiles [u][hk][dh][t] (4 consecutive t per lane -> one vector store).
  const int KV = HK * Dh;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + 16 * j + c16;
    const bool is_v = n >= KV;
    const int nn = is_v ? n - KV : n;
    const int hk = nn / Dh, dh = nn % Dh;
    T* dst = is_v ? vout : kout;
    T* dst_t = is_v ? vout_t : kout_t;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r0 = m0 + wm * 64 + 16 * i + 4 * g;
      T vals[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t r = r0 + e;
        vals[e] = from_f<T>(acc[i][j][e]);
        if (r < nrows) {
          const int64_t u = r / Tc, jj = r % Tc;
          if (dst) dst[((u * HK + hk) * Tc + jj) * Dh + dh] = vals[e];
        }
      }
      if (dst_t && r0 < nrows) {  // Tc % 32 == 0: the 4 rows share a chapter and stay adjacent in key order
        const int64_t u = r0 / Tc, jj = r0 % Tc;
        T* p = dst_t + ((u * HK + hk) * Dh + dh) * Tc + mfma_key_pos((int)jj);
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<bf16x4*>(p) = bf16x4{vals[0], vals[1], vals[2], vals[3]};
        } else {
          *reinterpret_cast<f32x4*>(p) = f32x4{vals[0], vals[1], vals[2], vals[3]};
        }
      }
    }
  }
}


// Wide variant for bf16 compute with 64-row chapters and head_dim 64 (every caller
// of the attention kernels): 256 x 256 output tile per workgroup, 8 waves in a
// 2 (rows) x 4 (columns) grid of 128 x 64, so each wave owns two whole (chapter,
// head) 64 x 64 output blocks.  The k-stage is 64 columns (128 bytes) of A and B,
// double-buffered (128 KB of LDS).  The epilogue stages each block through the
// wave's own 16 KB of LDS (row-major and transposed copies) and writes every
// layout with 16-byte stores, one contiguous kilobyte per wave instruction.
constexpr int kWideThreads = 512;

template <typename TB, bool kNorm>
__global__ __launch_bounds__(kWideThreads) void kv_project_wide_kernel(
    const TB* __restrict__ bank, int64_t d, const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq,
    int64_t max_u, const float* __restrict__ row_mean, const float* __restrict__ row_rstd,
    const bf16* __restrict__ wkv, int HK, int n_mblk, int n_nblk, bf16* __restrict__ kout, bf16* __restrict__ vout,
    bf16* __restrict__ kout_t, bf16* __restrict__ vout_t) {
  using Tile = SwzTile<bf16, 64>;
  constexpr int STAGE = 256 * 128;  // one operand stage: 256 rows x 128 bytes
  constexpr bool kConv = kNorm || !std::is_same<TB, bf16>::value;
  constexpr int NV = (8 * (int)sizeof(TB)) / 16;  // 16-byte loads per 8-element A chunk
  __shared__ __attribute__((aligned(16))) char lds[2][2][STAGE];

  // XCD-aware raster (see kv_project_kernel)
  const int w = blockIdx.x, per = (int)(gridDim.x / 8);
  const int t = (w % 8) * per + w / 8;
  if (t >= n_mblk * n_nblk) return;
  const int nu = (int)min((int64_t)n_uniq[0], max_u);
  const int64_t nrows = (int64_t)nu * 64;
  const int64_t m0 = (int64_t)(t / n_nblk) * 256;
  if (m0 >= nrows) return;
  const int n0 = (t % n_nblk) * 256;
  const int KV = HK * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int g = lane >> 4, c16 = lane & 15;

  // staging: thread moves chunks q = tid + 512 i (i < 4) of A and of B (row q / 8, 16-byte column q % 8)
  const TB* a_src[4];
  float a_mu[4], a_rs[4];
  bool a_ok[4];
  int s_off[4];
  uint32_t b_off[4];
  // rows of W past 2 * HK * 64 read as zeros (buffer bound)
  const Buf wb(wkv, (uint32_t)((size_t)2 * KV * d * sizeof(bf16)));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + kWideThreads * i;
    const int row = q >> 3, cc = q & 7;
    const int64_t r = m0 + row;
    a_ok[i] = r < nrows;
    const int64_t rr = a_ok[i] ? r : 0;
    const int64_t src = (int64_t)uniq[rr >> 6] * 64 + (rr & 63);
    a_src[i] = bank + src * d + cc * 8;
    a_mu[i] = kNorm ? row_mean[rr] : 0.f;
    a_rs[i] = kNorm ? row_rstd[rr] : 1.f;
    s_off[i] = Tile::off(row, cc * 8);
    b_off[i] = (uint32_t)(((int64_t)(n0 + row) * d + cc * 8) * (int64_t)sizeof(bf16));
  }
  V16 ra[4][NV], rb[4];
  auto fetch = [&](int kt) {
    const int64_t ko = (int64_t)kt * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int x = 0; x < NV; ++x) ra[i][x] = ld16(a_src[i] + ko + x * (16 / (int)sizeof(TB)));
      rb[i] = wb.load16(b_off[i], (uint32_t)(kt * 128));
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      V16 av;
      if constexpr (!kConv) {
        av = a_ok[i] ? ra[i][0] : V16{{0u, 0u, 0u, 0u}};
      } else {
        float v[8];
        ChunkLoad<bf16, TB>::run(reinterpret_cast<const TB*>(ra[i]), v);
        bf16x8 o;
#pragma unroll
        for (int x = 0; x < 8; ++x) o[x] = (bf16)(a_ok[i] ? (v[x] - a_mu[i]) * a_rs[i] : 0.f);
        av = __builtin_bit_cast(V16, o);
      }
      st16(&lds[buf][0][s_off[i]], av);
      st16(&lds[buf][1][s_off[i]], rb[i]);
    }
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)(d / 64);
  fetch(0);
  stash(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) fetch(kt + 1);
    const char* As = lds[buf][0];
    const char* Bs = lds[buf][1];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Tile::frag(Bs, 64 * wn + 16 * j + c16, 32 * ks + 8 * g);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bf16x8 a = Tile::frag(As, 128 * wm + 16 * i + c16, 32 * ks + 8 * g);
#pragma unroll
        for (int j = 0; j < 4; ++j) mma(acc[i][j], a, b[j]);
      }
    }
    if (kt + 1 < nk) stash(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: this wave's columns are one head of K or V
  const int col0 = n0 + 64 * wn;
  if (col0 >= 2 * KV) return;
  const bool is_v = col0 >= KV;
  const int hk = (is_v ? col0 - KV : col0) / 64;
  bf16* dst = is_v ? vout : kout;
  bf16* dst_t = is_v ? vout_t : kout_t;
  char* R = &lds[0][0][0] + wave * 16384;  // [t][dh] block
  char* Rt = R + 8192;                       // [dh][t] block
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int64_t u = (m0 + 128 * wm + 64 * blk) >> 6;
    if (u >= nu) break;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * blk + ii;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tt = 16 * ii + 4 * g, dh = 16 * j + c16;
        const bf16x4 v4 = bf16x4{(bf16)acc[i][j][0], (bf16)acc[i][j][1], (bf16)acc[i][j][2], (bf16)acc[i][j][3]};
        if (dst) {
#pragma unroll
          for (int e = 0; e < 4; ++e) *reinterpret_cast<bf16*>(R + Tile::off(tt + e, dh)) = v4[e];
        }
        if (dst_t) *reinterpret_cast<bf16x4*>(Rt + Tile::off(dh, mfma_key_pos(tt))) = v4;  // 4 keys stay adjacent
      }
    }
    __builtin_amdgcn_wave_barrier();
    const size_t base = ((size_t)u * HK + hk) * 4096;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int ch = lane + 64 * m, row = ch >> 3, c8 = (ch & 7) * 8;
      if (dst) st16(dst + base + row * 64 + c8, ld16(R + Tile::off(row, c8)));
      if (dst_t) st16(dst_t + base + row * 64 + c8, ld16(Rt + Tile::off(row, c8)));
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_row_stats(const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq, const int32_t* n_uniq,
                  int64_t max_u, int norm, float eps, float* mean, float* rstd, hipStream_t stream) {
  MOC_REQUIRE(bank && uniq && n_uniq && mean && rstd, MOC_ERR_ARG, "moc_row_stats: null pointer");
  MOC_REQUIRE(norm == MOC_NORM_RMS || norm == MOC_NORM_LAYERNORM, MOC_ERR_ARG, "moc_row_stats: norm=%d", norm);
  MOC_REQUIRE(d > 0 && T > 0 && max_u >= 0, MOC_ERR_ARG, "moc_row_stats: bad shape");
  if (max_u == 0) return MOC_OK;
  const int64_t rows = max_u * T;
  dim3 grid((unsigned)((rows + 3) / 4));
  if (bank_dtype == MOC_F32)
    hipLaunchKernelGGL(row_stats_kernel<float>, grid, dim3(256), 0, stream, (const float*)bank, d, T, uniq, n_uniq, max_u,
                       norm, eps, mean, rstd);
  else if (bank_dtype == MOC_BF16)
    hipLaunchKernelGGL(row_stats_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)bank, d, T, uniq, n_uniq, max_u,
                       norm, eps, mean, rstd);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_row_stats: dtype %d", bank_dtype);
  return check_launch("row_stats_kernel");
}

int moc_kv_project(int dtype, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                   const int32_t* n_uniq, int64_t max_u, const float* row_mean, const float* row_rstd,
                   const void* wkv, int HK, int Dh, void* k_tiles, void* v_tiles, void* kt_tiles, void* vt_tiles,
                   hipStream_t stream) {
  MOC_REQUIRE(bank && uniq && n_uniq && wkv && (k_tiles || kt_tiles) && (v_tiles || vt_tiles), MOC_ERR_ARG,
              "moc_kv_project: null pointer");
  MOC_REQUIRE((row_mean == nullptr) == (row_rstd == nullptr), MOC_ERR_ARG, "moc_kv_project: mean/rstd must be both set or both null");
  MOC_REQUIRE(T > 0 && HK > 0 && Dh > 0 && max_u >= 0, MOC_ERR_ARG, "moc_kv_project: bad shape");
  MOC_REQUIRE((kt_tiles == nullptr && vt_tiles == nullptr) || T % 32 == 0, MOC_ERR_ARG,
              "moc_kv_project: transposed tiles need T %% 32 == 0");
  const int BK = dtype == MOC_BF16 ? 64 : 32;
  MOC_REQUIRE(d % 64 == 0 && d >= BK, MOC_ERR_UNSUPPORTED, "moc_kv_project: memory_dim %lld must be a multiple of 64",
              (long long)d);
  MOC_REQUIRE((2 * HK * Dh) % 128 == 0, MOC_ERR_UNSUPPORTED, "moc_kv_project: 2*HK*Dh=%d must be a multiple of 128",
              2 * HK * Dh);
  if (max_u == 0) return MOC_OK;
  const int64_t rows = max_u * T;
  if (dtype == MOC_BF16 && T == 64 && Dh == 64) {
    const int64_t n_mblk = (rows + 255) / 256, n_nblk = (2 * HK * Dh + 255) / 256;
    MOC_REQUIRE(n_mblk * n_nblk < ((int64_t)1 << 30) && 2 * HK * Dh * d * 2 < ((int64_t)1 << 32),
                MOC_ERR_UNSUPPORTED, "moc_kv_project: problem too large");
    const int64_t n_tiles = n_mblk * n_nblk;
    dim3 grid((unsigned)((n_tiles + 7) / 8 * 8));  // a multiple of the 8 XCDs
    const bool norm = row_rstd != nullptr;
#define MOC_KVW(TB, NORM)                                                                                        \
  hipLaunchKernelGGL((kv_project_wide_kernel<TB, NORM>), grid, dim3(kWideThreads), 0, stream, (const TB*)bank, d, \
                     uniq, n_uniq, max_u, row_mean, row_rstd, (const bf16*)wkv, HK, (int)n_mblk, (int)n_nblk,     \
                     (bf16*)k_tiles, (bf16*)v_tiles, (bf16*)kt_tiles, (bf16*)vt_tiles)
    if (bank_dtype == MOC_BF16) {
      if (norm) MOC_KVW(bf16, true); else MOC_KVW(bf16, false);
    } else if (bank_dtype == MOC_F32) {
      if (norm) MOC_KVW(float, true); else MOC_KVW(float, false);
    } else {
      return set_error(MOC_ERR_UNSUPPORTED, "moc_kv_project: bank dtype %d", bank_dtype);
    }
#undef MOC_KVW
    return check_launch("kv_project_wide_kernel");
  }
  const int64_t n_mblk = (rows + 127) / 128, n_nblk = 2 * HK * Dh / 128;
  MOC_REQUIRE(n_mblk * n_nblk < ((int64_t)1 << 30), MOC_ERR_UNSUPPORTED, "moc_kv_project: too many tiles");
  const int64_t n_tiles = n_mblk * n_nblk;
  dim3 grid((unsigned)((n_tiles + 7) / 8 * 8));  // a multiple of the 8 XCDs
  if (dtype == MOC_BF16 && bank_dtype == MOC_BF16)
    hipLaunchKernelGGL((kv_project_kernel<bf16, bf16>), grid, dim3(kGemmThreads), 0, stream, (const bf16*)bank, d, T, uniq,
                       n_uniq, max_u, row_mean, row_rstd, (const bf16*)wkv, HK, Dh, (int)n_mblk, (int)n_nblk, (bf16*)k_tiles, (bf16*)v_tiles, (bf16*)kt_tiles, (bf16*)vt_tiles);
  else if (dtype == MOC_BF16 && bank_dtype == MOC_F32)
    hipLaunchKernelGGL((kv_project_kernel<bf16, float>), grid, dim3(kGemmThreads), 0, stream, (const float*)bank, d, T, uniq,
                       n_uniq, max_u, row_mean, row_rstd, (const bf16*)wkv, HK, Dh, (int)n_mblk, (int)n_nblk, (bf16*)k_tiles, (bf16*)v_tiles, (bf16*)kt_tiles, (bf16*)vt_tiles);
  else if (dtype == MOC_F32 && bank_dtype == MOC_F32)
    hipLaunchKernelGGL((kv_project_kernel<float, float>), grid, dim3(kGemmThreads), 0, stream, (const float*)bank, d, T,
                       uniq, n_uniq, max_u, row_mean, row_rstd, (const float*)wkv, HK, Dh, (int)n_mblk, (int)n_nblk, (float*)k_tiles,
                       (float*)v_tiles, (float*)kt_tiles, (float*)vt_tiles);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_kv_project: dtype %d with bank dtype %d", dtype, bank_dtype);
  return check_launch("kv_project_kernel");
}

}  // extern "C"
