// Weight gradient of the K/V projection, with the chapter gather fused in.
//
//   dW[n, k] = sum_r dkv[r, n] * X[r, k]      n < 2*HK*Dh, k < d, r < n_uniq * 64
//   X[r, :]  = norm(bank[uniq[r / 64] * 64 + r % 64, :])
//
// This is the weight gradient of k_proj / v_proj (memory_transformer/
// memory_attention.py:241-243, nn.Linear) over the gathered, normalised memory
// rows (memory_transformer/memory_bank.py:263-293, model.py:393-432); the
// reference gets it from autograd.  The reduction runs over ~32k rows while the
// output is only 2*HK*Dh x d, so the rows are split over `splits` workgroups per
// 256 x 256 output tile; each writes an fp32 partial tile and
// kv_wgrad_reduce_kernel sums the partials in a fixed order (deterministic).
//
// Both operands have the reduction index (rows r) outermost in memory.  They are
// staged in LDS in their natural [r][column] layout and the MFMA fragments (8
// consecutive r per lane) are read with gfx950's transposing LDS load
// ds_read_b64_tr_b16: within each 16-lane group, lane q supplies the address of
// row q / 4, columns 4 (q % 4) .. +3, and lane i receives column i of those four
// rows.  Two such loads give a lane its 8 rows of one column.
#include "moc_common.h"

#include <type_traits>

namespace moc {

constexpr int kWgThreads = 512;

// [64 rows][256 bf16] stage tile, 512-byte rows: 16-byte chunk c of row r sits
// at c ^ s(r) with s(r) = (r & 3) | ((r >> 3) & 3) << 2, which spreads the 16
// rows touched by one transposing load (r = 8 g + q, g, q < 4) over 16 distinct
// bank groups.
struct WgTile {
  __device__ static __forceinline__ int off(int row, int col) {
    const int s = (row & 3) | (((row >> 3) & 3) << 2);
    return row * 512 + ((((col >> 3) ^ s) & 31) << 4) + ((col & 7) << 1);
  }
};

typedef short v4s_t __attribute__((ext_vector_type(4)));

// MFMA fragment: rows rb + 8 g + 0..7 (g = lane / 16) of column cb + lane % 16
__device__ __forceinline__ bf16x8 tr_frag(const char* base, int rb, int cb, int lane) {
  const int q = lane & 15;
  const int row = rb + 8 * (lane >> 4) + (q >> 2), col = cb + 4 * (q & 3);
  typedef __attribute__((address_space(3))) v4s_t* lds_v4s;
  const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + WgTile::off(row, col)));
  const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + WgTile::off(row + 4, col)));
  const v4s_t v[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8, v);
}

// kGather: X rows are gathered chapter rows (stage st = distinct chapter st); otherwise X
// is a dense [R][d] matrix and stage st covers rows 64 st .. 64 st + 63 (rows >= R read zero).
template <typename TB, bool kNorm, bool kGather>
__global__ __launch_bounds__(kWgThreads) void kv_wgrad_kernel(
    const bf16* __restrict__ dkv, int KV2, const TB* __restrict__ bank, int64_t d, const int32_t* __restrict__ uniq,
    const int32_t* __restrict__ n_uniq, const int32_t* __restrict__ edge_u, int64_t max_u, int64_t R,
    const float* __restrict__ row_mean,
    const float* __restrict__ row_rstd, int n_ktile, int n_tiles, int splits, float* __restrict__ ws) {
  constexpr int STAGE = 64 * 512;
  constexpr bool kConv = kNorm || !std::is_same<TB, bf16>::value;
  constexpr int NV = (8 * (int)sizeof(TB)) / 16;
  __shared__ __attribute__((aligned(16))) char lds[2][2][STAGE];  // [buf][dkv | X]

  // (split, tile) with split major, so the tiles that read the same rows share an XCD
  const int64_t t = xcd_tile((int64_t)n_tiles * splits);
  if (t < 0) return;
  const int tile = (int)(t % n_tiles), split = (int)(t / n_tiles);
  const int n0 = (tile / n_ktile) * 256, k0 = (tile % n_ktile) * 256;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 2, wk = wave & 3;  // wave tile: 128 (n) x 64 (k)
  const int g = lane >> 4, c16 = lane & 15;

  // one 64-row stage per distinct chapter (gather), per edge (gather with edge_u: dkv rows are
  // per edge, e -> distinct chapter edge_u[e], skipped edges read as zero) or per 64 rows (dense)
  const int64_t nstage = !kGather ? (R + 63) / 64 : edge_u ? max_u : (int64_t)min((int64_t)n_uniq[0], max_u);
  const int64_t per = (nstage + splits - 1) / splits;
  const int64_t s0 = min(nstage, (int64_t)split * per), s1 = min(nstage, s0 + per);

  // staging: chunks q = tid + 512 i (i < 4) of each operand: row q / 32, 16-byte column q % 32
  int s_off[4];
  bool a_ok[4], b_ok[4];
  const bf16* a_src[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + kWgThreads * i;
    const int row = q >> 5, cc = (q & 31) * 8;
    s_off[i] = WgTile::off(row, cc);
    a_ok[i] = n0 + cc < KV2;
    b_ok[i] = k0 + cc < d;
    a_src[i] = dkv + (int64_t)row * KV2 + (a_ok[i] ? n0 + cc : 0);
  }
  V16 ra[4], rb[4][NV];
  float mu[4], rs[4];
  auto fetch = [&](int64_t st) {
    // distinct chapter of the stage (-1: a skipped edge) and its first X row
    const int64_t u = !kGather ? 0 : edge_u ? (int64_t)edge_u[st] : st;
    const int64_t xbase = !kGather ? st * 64 : u >= 0 ? (int64_t)uniq[u] * 64 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + kWgThreads * i;
      const int row = q >> 5, cc = (q & 31) * 8;
      const bool live = kGather ? u >= 0 : st * 64 + row < R;
      ra[i] = a_ok[i] && live ? ld16(a_src[i] + st * 64 * KV2) : V16{{0u, 0u, 0u, 0u}};
      const TB* xp = bank + (xbase + row) * d + (b_ok[i] ? k0 + cc : 0);
#pragma unroll
      for (int x = 0; x < NV; ++x)
        rb[i][x] = b_ok[i] && live ? ld16(xp + x * (16 / (int)sizeof(TB))) : V16{{0u, 0u, 0u, 0u}};
      if constexpr (kNorm) {
        mu[i] = live ? row_mean[u * 64 + row] : 0.f;
        rs[i] = live ? row_rstd[u * 64 + row] : 0.f;
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st16(&lds[buf][0][s_off[i]], ra[i]);
      V16 xv;
      if constexpr (!kConv) {
        xv = rb[i][0];
      } else {
        float v[8];
        ChunkLoadF<TB>::run(reinterpret_cast<const TB*>(rb[i]), v);
        bf16x8 o;
#pragma unroll
        for (int x = 0; x < 8; ++x) o[x] = (bf16)(kNorm ? (v[x] - mu[i]) * rs[i] : v[x]);
        xv = __builtin_bit_cast(V16, o);
      }
      st16(&lds[buf][1][s_off[i]], xv);
    }
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (s0 < s1) {
    fetch(s0);
    stash(0);
    __syncthreads();
    for (int64_t st = s0; st < s1; ++st) {
      const int buf = (int)((st - s0) & 1);
      if (st + 1 < s1) fetch(st + 1);
      const char* As = lds[buf][0];
      const char* Bs = lds[buf][1];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 bfr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bfr[j] = tr_frag(Bs, 32 * ks, 64 * wk + 16 * j, lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bf16x8 afr = tr_frag(As, 32 * ks, 128 * wn + 16 * i, lane);
#pragma unroll
          for (int j = 0; j < 4; ++j) mma(acc[i][j], afr, bfr[j]);
        }
      }
      if (st + 1 < s1) stash(buf ^ 1);
      __syncthreads();
    }
  }
  // partial tile in accumulator order: [split][tile][wave][i][j][lane] f32x4
  f32x4* out = reinterpret_cast<f32x4*>(ws) + (((size_t)split * n_tiles + tile) * 8 + wave) * 32 * 64 + lane;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) out[(i * 4 + j) * 64] = acc[i][j];
}

// dW[n, k] = sum over splits (in order) of the partial tiles; one thread per f32x4.
template <typename TO>
__global__ __launch_bounds__(256) void kv_wgrad_reduce_kernel(const float* __restrict__ ws, int splits, int n_tiles,
                                                              int n_ktile, int KV2, int64_t d, TO* __restrict__ dw) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;  // f32x4 index within one split
  const int64_t per_split = (int64_t)n_tiles * 8 * 32 * 64;
  if (p >= per_split) return;
  f32x4 s = reinterpret_cast<const f32x4*>(ws)[p];
  for (int sp = 1; sp < splits; ++sp) s += reinterpret_cast<const f32x4*>(ws)[sp * per_split + p];
  const int lane = (int)(p & 63), ij = (int)((p >> 6) & 31), wave = (int)((p >> 11) & 7);
  const int tile = (int)(p >> 14);
  const int i = ij >> 2, j = ij & 3, wn = wave >> 2, wk = wave & 3;
  const int n = (tile / n_ktile) * 256 + 128 * wn + 16 * i + 4 * (lane >> 4);
  const int64_t k = (int64_t)(tile % n_ktile) * 256 + 64 * wk + 16 * j + (lane & 15);
  if (k >= d) return;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (n + e < KV2) dw[(int64_t)(n + e) * d + k] = from_f<TO>(s[e]);
}

}  // namespace moc

namespace moc {
int chapter_wgrad_dense(const void* dy, const void* x, int64_t R, int64_t N, int64_t K, void* ws, int out_dtype,
                        void* dw, hipStream_t stream);
}

using namespace moc;

namespace {
int wgrad_tiles(int64_t KV2, int64_t d, int* n_ktile) {
  *n_ktile = (int)((d + 255) / 256);
  return (int)((KV2 + 255) / 256) * *n_ktile;
}
// workgroups per output tile: fill the 256 CUs, but give each at least 8 stages
int wgrad_splits(int tiles, int64_t max_stages) {
  int64_t s = 256 / tiles;
  const int64_t by_len = (max_stages + 7) / 8;
  if (s > by_len) s = by_len;
  if (s < 1) s = 1;
  return (int)s;
}

template <bool kGather>
int launch_wgrad(const void* dkv, const void* bank, int bank_dtype, int64_t d, const int32_t* uniq,
                 const int32_t* n_uniq, const int32_t* edge_u, int64_t max_u, int64_t R, const float* row_mean,
                 const float* row_rstd,
                 int64_t KV2, int64_t max_stages, void* ws, int out_dtype, void* dw, hipStream_t stream) {
  int nk;
  const int tiles = wgrad_tiles(KV2, d, &nk);
  const int splits = wgrad_splits(tiles, max_stages);
  MOC_REQUIRE(tiles < 65536 && splits < 65536, MOC_ERR_UNSUPPORTED, "weight gradient: problem too large");
  dim3 grid(xcd_grid((int64_t)tiles * splits));
  const bool norm = row_rstd != nullptr;
#define MOC_WG(TB, NORM)                                                                                        \
  hipLaunchKernelGGL((kv_wgrad_kernel<TB, NORM, kGather>), grid, dim3(kWgThreads), 0, stream, (const bf16*)dkv, \
                     (int)KV2, (const TB*)bank, d, uniq, n_uniq, edge_u, max_u, R, row_mean, row_rstd, nk, tiles,    \
                     splits, (float*)ws)
  if (bank_dtype == MOC_BF16) {
    if (norm) MOC_WG(bf16, true); else MOC_WG(bf16, false);
  } else if (bank_dtype == MOC_F32) {
    if (norm) MOC_WG(float, true); else MOC_WG(float, false);
  } else {
    return set_error(MOC_ERR_UNSUPPORTED, "weight gradient: input dtype %d", bank_dtype);
  }
#undef MOC_WG
  int rc = check_launch("kv_wgrad_kernel");
  if (rc != MOC_OK) return rc;
  const int64_t n4 = (int64_t)tiles * 8 * 32 * 64;
  dim3 rgrid((unsigned)((n4 + 255) / 256));
  if (out_dtype == MOC_F32)
    hipLaunchKernelGGL(kv_wgrad_reduce_kernel<float>, rgrid, dim3(256), 0, stream, (const float*)ws, splits, tiles, nk,
                       (int)KV2, d, (float*)dw);
  else if (out_dtype == MOC_BF16)
    hipLaunchKernelGGL(kv_wgrad_reduce_kernel<bf16>, rgrid, dim3(256), 0, stream, (const float*)ws, splits, tiles, nk,
                       (int)KV2, d, (bf16*)dw);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "weight gradient: out dtype %d", out_dtype);
  return check_launch("kv_wgrad_reduce_kernel");
}
}  // namespace

extern "C" {

size_t moc_kv_wgrad_workspace(int64_t KV2, int64_t d, int64_t max_u) {
  int nk;
  const int tiles = wgrad_tiles(KV2, d, &nk);
  return (size_t)wgrad_splits(tiles, max_u) * tiles * 256 * 256 * sizeof(float);
}

int moc_kv_wgrad(const void* dkv, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                 const int32_t* n_uniq, const int32_t* edge_u, int64_t max_u, const float* row_mean,
                 const float* row_rstd, int64_t KV2, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                 hipStream_t stream) {
  MOC_REQUIRE(dkv && bank && uniq && n_uniq && ws && dw, MOC_ERR_ARG, "moc_kv_wgrad: null pointer");
  MOC_REQUIRE((row_mean == nullptr) == (row_rstd == nullptr), MOC_ERR_ARG,
              "moc_kv_wgrad: mean/rstd must be both set or both null");
  MOC_REQUIRE(T == 64, MOC_ERR_UNSUPPORTED, "moc_kv_wgrad: needs 64 tokens per chapter (got %d)", T);
  MOC_REQUIRE(d > 0 && d % 8 == 0 && KV2 > 0 && KV2 % 8 == 0 && KV2 < (1 << 30) && max_u >= 0, MOC_ERR_UNSUPPORTED,
              "moc_kv_wgrad: d=%lld KV2=%lld must be multiples of 8", (long long)d, (long long)KV2);
  MOC_REQUIRE(ws_bytes >= moc_kv_wgrad_workspace(KV2, d, max_u), MOC_ERR_ARG, "moc_kv_wgrad: workspace too small");
  return launch_wgrad<true>(dkv, bank, bank_dtype, d, uniq, n_uniq, edge_u, max_u, 0, row_mean, row_rstd, KV2, max_u,
                            ws, out_dtype, dw, stream);
}

size_t moc_linear_wgrad_workspace(int64_t R, int64_t N, int64_t K) {
  int nk;
  const int tiles = wgrad_tiles(N, K, &nk);
  return (size_t)wgrad_splits(tiles, (R + 63) / 64) * tiles * 256 * 256 * sizeof(float);
}

int moc_linear_wgrad(const void* dy, const void* x, int x_dtype, int64_t R, int64_t N, int64_t K, void* ws,
                     size_t ws_bytes, int out_dtype, void* dw, hipStream_t stream) {
  MOC_REQUIRE(dy && x && ws && dw, MOC_ERR_ARG, "moc_linear_wgrad: null pointer");
  MOC_REQUIRE(R >= 0 && N > 0 && N % 8 == 0 && N < (1 << 30) && K > 0 && K % 8 == 0, MOC_ERR_UNSUPPORTED,
              "moc_linear_wgrad: N=%lld K=%lld must be multiples of 8", (long long)N, (long long)K);
  MOC_REQUIRE(ws_bytes >= moc_linear_wgrad_workspace(R, N, K), MOC_ERR_ARG, "moc_linear_wgrad: workspace too small");
  MOC_REQUIRE(out_dtype == MOC_F32 || out_dtype == MOC_BF16, MOC_ERR_UNSUPPORTED, "moc_linear_wgrad: out dtype %d",
              out_dtype);
  // bf16 operands on 256-multiples: the LDS-DMA chapter weight-gradient kernel (same splits)
  if (x_dtype == MOC_BF16 && N % 256 == 0 && K % 256 == 0 && R > 0 && R * (N > K ? N : K) * 2 < ((int64_t)1 << 40))
    return chapter_wgrad_dense(dy, x, R, N, K, ws, out_dtype, dw, stream);
  return launch_wgrad<false>(dy, x, x_dtype, K, nullptr, nullptr, nullptr, 0, R, nullptr, nullptr, N, (R + 63) / 64,
                             ws, out_dtype, dw, stream);
}

}  // extern "C"
