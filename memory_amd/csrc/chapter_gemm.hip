// Chapter-block GEMMs of the K/V path on the matrix cores.
//
//   Y_c[j, n] = sum_k X_c[j, k] * W[n, k]      for every distinct chapter c < n_uniq, j < 64
//
// X_c is a block of 64 rows chosen per chapter (the chapter's bank rows, a contiguous block, or
// the chapter's per-edge dK/dV rows), W is [N][K] bf16, and Y_c is stored to a block chosen per
// chapter (contiguous projection rows, or the chapter's rows of the bank gradient).  Two uses:
//
//  * moc_chapter_project: K/V projection of the distinct chapters, gather fused into the operand
//    loads (memory_transformer/memory_bank.py:263-293 get_chapters_batched, then k_proj / v_proj
//    of memory_attention.py:241-243 with W = [Wk; Wv]).  The router weight omega is applied
//    inside attention ((omega x) W^T = omega (x W^T)), so one projected chapter serves every
//    sequence that selected it.
//  * moc_chapter_dx: the input gradient of that projection summed over a chapter's edges and
//    stored into the chapter's bank rows (the autograd of k_proj / v_proj followed by the
//    scatter-add of the gather's backward, memory_bank.py:287-291): W = [Wk; Wv]^T, X_c = the
//    chapter's dK|dV rows (one edge) or their sum (several edges, summed beforehand by
//    dkv_multi_reduce_kernel), stores straight into the dense bank gradient (distinct chapters
//    own distinct rows, so no atomics).
//
// Kernel design (gfx950): a persistent grid of one 512-thread workgroup per CU walks a list of
// BN (features) x BM (rows) output tiles: 256 x 384 for the K/V projection and its dX (2 x 80 KB
// of LDS: a sixth less operand traffic per product than 256 x 256, which measured 86 / 102 us
// against 82 / 76 us at c3), 128 x 256 for the dense rows GEMMs.  Each XCD (workgroups are dealt
// round-robin to the 8 XCDs) takes a contiguous range of tiles, feature blocks fastest, so the
// feature tiles of one row block share its X rows in that XCD's L2.  Operands move global -> LDS
// with buffer_load ... lds (no VGPR staging), 64 k-columns per stage, DEPTH stages loaded ahead
// of the one being computed (DEPTH + 1 LDS buffers per operand: 2 for 256-row tiles, 3 for
// 128-row tiles, whose few tiles per workgroup leave nothing else to hide the load latency); the
// 16-byte chunks of every LDS row are XOR-swizzled by (row & 7) so fragment reads are
// conflict-free.  8 waves in a 4 (features) x 2 (rows) grid; each wave owns BN/4 features x BM/2
// rows (v_mfma_f32_16x16x32_bf16, fp32 accumulators in VGPRs: 192 of them at BN 384).  The W
// tile's rows sit in LDS in a permuted order (row 32b + 16h + 4g + e holds feature 32b + 8g + 4h +
// e) so that a lane's accumulators of two adjacent MFMA tiles are 8 consecutive features of one
// row: the epilogue writes every output row piece with one 16-byte store (bf16) straight from
// registers.
#include "moc_common.h"

namespace moc {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kCgThreads = 512;
constexpr int kCgDxRows = 128;        // row tile of the dX GEMM (N = d is 3 feature tiles at d = 768)
constexpr int kCgDepth256 = 1;        // k-stages loaded ahead with 256-row tiles (LDS: 2 x 64 KB, 2 x 80 KB at BN 384)
constexpr int kCgDepth128 = 2;        // ... with 128-row tiles (LDS: 3 x 48 KB)

enum { CG_SRC_GATHER = 0, CG_SRC_CONTIG = 1, CG_SRC_EDGE = 2 };
enum { CG_DST_CONTIG = 0, CG_DST_BANK = 1 };

__device__ __forceinline__ int cg_perm(int r) {
  return (r & ~31) | (((r >> 2) & 3) << 3) | (((r >> 4) & 1) << 2) | (r & 3);
}

__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }

// 8 consecutive elements as floats (one 16-byte load for bf16, two for f32)
template <typename T> struct ChunkLoad8;
template <> struct ChunkLoad8<bf16> {
  static __device__ __forceinline__ void run(const bf16* p, float* o) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int x = 0; x < 8; ++x) o[x] = (float)v[x];
  }
};
template <> struct ChunkLoad8<float> {
  static __device__ __forceinline__ void run(const float* p, float* o) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int x = 0; x < 4; ++x) { o[x] = a[x]; o[4 + x] = b[x]; }
  }
};

// buffer resource over `bytes` bytes at p (raw buffer, bounds-checked; a macro, since the
// host pass of the kernel templates cannot take the resource type through a function)
#define CG_RSRC(p, bytes) \
  __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>((const void*)(p)), (short)0, (int)(bytes), 0x00020000)


template <int SRC>
__device__ __forceinline__ const bf16* cg_src_rows(int c, const bf16* __restrict__ x, const bf16* __restrict__ xred,
                                                   int64_t ldx, const int32_t* __restrict__ uniq,
                                                   const int32_t* __restrict__ csr_off,
                                                   const int32_t* __restrict__ csr_edge) {
  if constexpr (SRC == CG_SRC_GATHER) {
    return x + (int64_t)rfl(uniq[c]) * 64 * ldx;
  } else if constexpr (SRC == CG_SRC_CONTIG) {
    return x + (int64_t)c * 64 * ldx;
  } else {
    const int p0 = rfl(csr_off[c]), cnt = rfl(csr_off[c + 1]) - p0;
    return cnt == 1 ? x + (int64_t)rfl(csr_edge[p0]) * 64 * ldx : xred + (int64_t)c * 64 * ldx;
  }
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes at voff (+ soff)
// of the buffer land at LDS address m0 + 16 l.  Written as inline assembly so that the waits
// on these loads stay explicit (cg_wait_vm): the compiler's own accounting waits for every
// outstanding load and store before each barrier, which would also wait for the loads issued
// ahead for later stages and for the epilogue's stores.
__device__ __forceinline__ void cg_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const char* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0) : "memory");
}
// s_waitcnt vmcnt(n), n in {0, 5, 6, 8}: all but this wave's newest n vector memory operations
// done (loads complete in issue order); any other n waits for everything
__device__ __forceinline__ void cg_wait_vm(int n) {
  if (n == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if (n == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if (n == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Row normalisation folded into the rows GEMM (NORM = MOC_NORM_RMS or MOC_NORM_LAYERNORM): y =
// norm(x) W^T with W already scaled by the norm weight (moc_norm_fold_weight) is
// rstd (x W~^T) for RMSNorm and rstd (x W~^T - mean u) + v for LayerNorm (u = W~ 1, v = W beta),
// so the GEMM reads the raw rows; each row's sums of x and x^2 are taken from the X tiles the
// stages bring into LDS anyway (4 threads per row, 16 columns each, by bf16 dot2) and applied
// in the epilogue.
struct CgNorm {
  float eps;
  const float* u;   // LayerNorm: [N]
  const float* v;   // LayerNorm: [N]
  float* mean_out;  // LayerNorm: [rows] or null
  float* rstd_out;  // [rows] or null
};

// Epilogue options of the contiguous rows GEMM (bit flags): EPI_RES adds residual rows (bf16, the
// output's row indexing, row stride ldr) to the fp32 product before the one rounding to bf16;
// EPI_BIAS adds a per-feature f32 bias; EPI_MASKN allows any N (the W rows past N read zero, the
// output columns past N are not stored; fp32 output by element stores, so any row stride).
enum { CG_EPI_RES = 1, CG_EPI_BIAS = 2, CG_EPI_MASKN = 4 };
struct CgEpi {
  const bf16* res;
  int64_t ldr;
  const float* bias;
};

template <int SRC, int DST, typename TO, int BM, int DEPTH, int NORM = MOC_NORM_NONE, int BN = 256, int EPI = 0>
__global__ __launch_bounds__(kCgThreads) void chapter_gemm_kernel(
    const bf16* __restrict__ x, const bf16* __restrict__ xred, int64_t ldx, const int32_t* __restrict__ uniq,
    const int32_t* __restrict__ n_uniq, const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge,
    int64_t max_u, const bf16* __restrict__ w, int N, int K, TO* __restrict__ y, int64_t ldy, int64_t xrows,
    int64_t yrows, CgNorm nrm = CgNorm{}, CgEpi ep = CgEpi{}) {
  static_assert(NORM == MOC_NORM_NONE || (SRC == CG_SRC_CONTIG && DST == CG_DST_CONTIG && BM == 128 &&
                                          sizeof(TO) == 2),
                "row normalisation: contiguous rows, 128-row tiles, bf16 output");
  static_assert(BN == 256 || BN == 384, "feature tile");
  static_assert(EPI == 0 || (SRC == CG_SRC_CONTIG && DST == CG_DST_CONTIG && NORM == MOC_NORM_NONE),
                "epilogue options: contiguous rows GEMM");
  static_assert(!(EPI & CG_EPI_RES) || sizeof(TO) == 2, "residual rows: bf16 output");
  static_assert(!(EPI & (CG_EPI_BIAS | CG_EPI_MASKN)) || sizeof(TO) == 4, "bias / any N: fp32 output");
  static_assert(!(EPI & CG_EPI_MASKN) || BN == 256, "any N: 256-feature tiles");
  constexpr int CPT = BM / 64;              // chapters per tile
  constexpr int IPX = BM / 64;              // X DMA instructions per thread per stage
  constexpr int FT = BN / 64;               // 16-feature MFMA tiles per wave (= W DMA instructions per thread)
  constexpr int JB = BM / 32;               // 16-row MFMA tiles per wave
  constexpr int STW = BN * 128;             // LDS bytes of one W stage (BN rows x 64 bf16)
  constexpr int STX = BM * 128;             // LDS bytes of one X stage
  constexpr int NBUF = DEPTH + 1;           // LDS buffers per operand
  constexpr int kBatch = FT + IPX;          // DMA instructions per wave and stage (W, then X)
  // any N: each wave's 16-row x 64-feature fp32 output block is staged in 4 KB of LDS so that the
  // stores go out as whole row pieces (element stores: any row stride)
  constexpr int EPI_LDS = (EPI & CG_EPI_MASKN) ? 8 * 4096 : 0;
  static_assert(NBUF * (STW + STX) + EPI_LDS <= 163840, "LDS");
  static_assert(DEPTH >= 1 && (DEPTH == 1 || (DEPTH - 1) * kBatch == 5 || (DEPTH - 1) * kBatch == 6 ||
                               (DEPTH - 1) * kBatch == 8), "cg_wait_vm count");
  __shared__ __attribute__((aligned(1024))) char smem[NBUF * (STW + STX) + EPI_LDS];
  char* const sW = smem;
  char* const sX = smem + NBUF * STW;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = rfl(tid >> 6);
  const int nu = n_uniq ? rfl((int)min((int64_t)n_uniq[0], max_u)) : (int)max_u;
  const int NB = (EPI & CG_EPI_MASKN) ? (N + BN - 1) / BN : N / BN;
  const int V = ((nu + CPT - 1) / CPT) * NB;  // tiles: row blocks x feature blocks
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nslot = gridDim.x >> 3;
  const int lo = (int)(((int64_t)xcd * V) >> 3), hi = (int)(((int64_t)(xcd + 1) * V) >> 3);
  const int nmine = hi - lo > slot ? (hi - lo - slot + nslot - 1) / nslot : 0;
  if (nmine == 0) return;
  const int nk = K >> 6;
  const int S = nmine * nk;  // stages of this workgroup

  // DMA geometry: instruction i of wave w fills LDS rows 64 i + 8 w + lane / 8 (1 KB per
  // instruction), physical chunk lane % 8 holding logical chunk (lane % 8) ^ (row & 7).
  const int srow = 8 * wave + (lane >> 3);
  const int lchunk = (lane & 7) ^ (srow & 7);
  // cg_perm keeps bits >= 5, so W-tile row 64 i + srow holds feature 64 i + cg_perm(srow)
  const uint32_t woff = (uint32_t)(cg_perm(srow) * K * 2 + lchunk * 16);
  const uint32_t xoff = (uint32_t)(srow * ldx * 2 + lchunk * 16);
  const uint32_t xbytes = (uint32_t)(64 * ldx * 2);

  // Load cursor: the tile, k-stage and LDS buffer of the next stage whose loads go out, advanced
  // one stage per issue.  The per-tile operands of the loads (the W block's buffer resource, the
  // X rows' resources) are formed once per tile, so the instructions between a barrier and its
  // DMAs are only the DMAs and their LDS addresses (the divisions and 64-bit address arithmetic
  // per stage had cost ~180 scalar instructions there, with the matrix cores idle).
  int ld_t = lo + slot, ld_kt = 0, ld_buf = 0;
  __amdgpu_buffer_rsrc_t ld_w;
  __amdgpu_buffer_rsrc_t ld_x[IPX];
  // gathered / per-edge X sources: looked up once per row block, and the workgroup's next tile's
  // a tile ahead of its first stage (plan lookups are dependent scalar loads: kept off the path
  // from a barrier to the DMAs that follow it)
  int cur_rb = -1, nxt_rb = -1;
  const bf16* cur_src[IPX];
  const bf16* nxt_src[IPX];
  auto lookup = [&](int rb, const bf16** out) {
#pragma unroll
    for (int i = 0; i < IPX; ++i)
      out[i] = cg_src_rows<SRC>(min(rb * CPT + i, nu - 1), x, xred, ldx, uniq, csr_off, csr_edge);
  };
  auto ld_tile = [&]() {
    const int t = ld_t, rb = t / NB, nb = t - rb * NB;
    // (any N: the rows of the last feature block past N read zero)
    ld_w = CG_RSRC(w + (int64_t)nb * BN * K, (uint32_t)(min(BN, N - nb * BN) * K * 2));
    if constexpr (SRC != CG_SRC_CONTIG) {
      if (rb != cur_rb) {
        if (rb == nxt_rb) {
#pragma unroll
          for (int i = 0; i < IPX; ++i) cur_src[i] = nxt_src[i];
        } else {
          lookup(rb, cur_src);
        }
        cur_rb = rb;
        const int tn = t + nslot;
        if (tn < hi && tn / NB != rb) {
          nxt_rb = tn / NB;
          lookup(nxt_rb, nxt_src);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < IPX; ++i) {
      const int c = min(rb * CPT + i, nu - 1);  // rows of chapters past n_uniq: computed, not stored
      const bf16* xb = SRC == CG_SRC_CONTIG ? cg_src_rows<SRC>(c, x, xred, ldx, uniq, csr_off, csr_edge) : cur_src[i];
      // a contiguous source ends at row xrows: rows past it read zero
      const uint32_t bytes = SRC == CG_SRC_CONTIG ? (uint32_t)(min((int64_t)64, xrows - (int64_t)c * 64) * ldx * 2) : xbytes;
      ld_x[i] = CG_RSRC(xb, bytes);
    }
  };
  ld_tile();
  // the loads of the stage at the cursor (W rows, then X rows, into buffer ld_buf), then the
  // cursor moves on; the row offset of instruction i rides in the per-lane offset, which the
  // buffer bound checks
  auto issue = [&]() {
    const uint32_t so = (uint32_t)(ld_kt * 128);
    const char* dw = sW + ld_buf * STW + wave * 1024;
#pragma unroll
    for (int i = 0; i < FT; ++i) cg_dma16(ld_w, woff + (uint32_t)(64 * i * K * 2), so, dw + 8192 * i);
    const char* dx = sX + ld_buf * STX + wave * 1024;
#pragma unroll
    for (int i = 0; i < IPX; ++i) cg_dma16(ld_x[i], xoff, so, dx + 8192 * i);
    ld_buf = ld_buf + 1 == NBUF ? 0 : ld_buf + 1;
    if (++ld_kt == nk) {
      ld_kt = 0;
      ld_t += nslot;
      if (ld_t < hi) ld_tile();
    }
  };

  const int wf = wave & 3, wr = wave >> 2;
  const int g = lane >> 4, m = lane & 15;
  // fragment reads: row base + 16 i + m (so row & 7 == m & 7), logical chunk 4 ks + g
  const int aoff0 = (16 * FT * wf + m) * 128 + ((g ^ (m & 7)) << 4);
  const int aoff1 = (16 * FT * wf + m) * 128 + (((4 + g) ^ (m & 7)) << 4);
  const int boff0 = ((BM / 2) * wr + m) * 128 + ((g ^ (m & 7)) << 4);
  const int boff1 = ((BM / 2) * wr + m) * 128 + (((4 + g) ^ (m & 7)) << 4);

  f32x4 acc[FT][JB];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // row statistics (NORM): thread t sums columns 16 (t % 4) .. +15 of tile row t / 4 of each
  // X stage; the four partial sums of a row are combined at the tile's end into sStat
  __shared__ float2 sStat[NORM != MOC_NORM_NONE ? BM : 1];
  float st_x = 0.f, st_xx = 0.f;
  // LayerNorm: the sums are taken around a pivot, the row's first element (read at the tile's
  // first stage), so var = E[(x - p)^2] - (E[x - p])^2 does not cancel for rows whose mean is
  // large against their spread; RMSNorm needs sum x^2 only (no cancellation)
  float st_p = 0.f;
  const int st_row = tid >> 2, st_part = tid & 3;
  auto stats_stage = [&](const char* sx, bool first) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    if constexpr (NORM == MOC_NORM_LAYERNORM) {
      if (first) st_p = (float)*reinterpret_cast<const __bf16*>(sx + st_row * 128 + ((st_row & 7) << 4));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int pc = (2 * st_part + h) ^ (st_row & 7);
      const bf16x8_t v8 = *reinterpret_cast<const bf16x8_t*>(sx + st_row * 128 + (pc << 4));
      if constexpr (NORM == MOC_NORM_LAYERNORM) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float dx = (float)v8[e] - st_p;
          st_x += dx;
          st_xx = fmaf(dx, dx, st_xx);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x2_t p2 = bf16x2_t{v8[2 * e], v8[2 * e + 1]};
          st_xx = __builtin_amdgcn_fdot2_f32_bf16(p2, p2, st_xx, false);
        }
      }
    }
  };
  // at a tile's last stage: per-row (mean, rstd) into sStat (and, for the tile's first feature
  // block, to mean_out / rstd_out); every wave then reads its rows' statistics in the epilogue
  auto stats_finish = [&](int t) {
    st_xx += __shfl_xor(st_xx, 1, 64);
    st_xx += __shfl_xor(st_xx, 2, 64);
    if constexpr (NORM == MOC_NORM_LAYERNORM) {
      st_x += __shfl_xor(st_x, 1, 64);
      st_x += __shfl_xor(st_x, 2, 64);
    }
    if (st_part == 0) {
      const float inv_k = 1.f / (float)K;
      const float dmean = NORM == MOC_NORM_LAYERNORM ? st_x * inv_k : 0.f;  // mean - pivot
      const float mean = st_p + dmean;
      const float var = NORM == MOC_NORM_LAYERNORM ? fmaxf(st_xx * inv_k - dmean * dmean, 0.f) : st_xx * inv_k;
      const float rstd = rsqrtf(var + nrm.eps);
      sStat[st_row] = float2{mean, rstd};
      const int rb = t / NB, nb = t - rb * NB;
      const int64_t row = (int64_t)rb * BM + st_row;
      if (nb == 0 && row < yrows) {
        if (nrm.rstd_out) nrm.rstd_out[row] = rstd;
        if (NORM == MOC_NORM_LAYERNORM && nrm.mean_out) nrm.mean_out[row] = mean;
      }
    }
    st_x = 0.f;
    st_xx = 0.f;
    __syncthreads();
  };

  auto compute = [&](const char* sw, const char* sx) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ao = ks ? aoff1 : aoff0, bo = ks ? boff1 : boff0;
      bf16x8 a[FT];
#pragma unroll
      for (int i = 0; i < FT; ++i) a[i] = *reinterpret_cast<const bf16x8*>(sw + ao + 2048 * i);
#pragma unroll
      for (int jh = 0; jh < JB / 4; ++jh) {
        bf16x8 b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const bf16x8*>(sx + bo + 2048 * (4 * jh + j));
#pragma unroll
        for (int i = 0; i < FT; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) mma(acc[i][4 * jh + j], a[i], b[j]);
      }
    }
  };

  // Epilogue: lane (g, m) of wave (wf, wr) holds, for row (BM/2) wr + 16 j + m of the tile,
  // features nb*BN + (BN/4) wf + 32 p + 8 g .. + 7 in acc[2p][j] (4) and acc[2p+1][j] (4).
  // Rows of chapters >= n_uniq fall outside their chapter's buffer range and are dropped.
  auto epilogue = [&](int t) {
    const int rb = t / NB, nb = t - rb * NB;
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int rt = (BM / 2) * wr + 16 * j;     // tile row of this 16-row group (wave-uniform)
      const int c = rb * CPT + rt / 64;
      const bool live = c < nu;
      const int cc = live ? c : 0;
      TO* dst = DST == CG_DST_BANK ? y + (int64_t)rfl(uniq[cc]) * 64 * ldy : y + (int64_t)cc * 64 * ldy;
      // a contiguous destination ends at row yrows: stores past it are dropped
      const int64_t yr = DST == CG_DST_CONTIG ? min((int64_t)64, yrows - (int64_t)cc * 64) : 64;
      const __amdgpu_buffer_rsrc_t yres = CG_RSRC(dst, live ? (uint32_t)(yr * ldy * sizeof(TO)) : 0u);
      const uint32_t vrow = (uint32_t)((((rt & 63) + m) * ldy + nb * BN + 16 * FT * wf + 8 * g) * sizeof(TO));
      __amdgpu_buffer_rsrc_t rres = yres;
      uint32_t rrow = 0;
      if constexpr ((EPI & CG_EPI_RES) != 0) {
        rres = CG_RSRC(ep.res + (int64_t)cc * 64 * ep.ldr, live ? (uint32_t)(yr * ep.ldr * 2) : 0u);
        rrow = (uint32_t)((((rt & 63) + m) * ep.ldr + nb * BN + 16 * FT * wf + 8 * g) * 2);
      }
#pragma unroll
      for (int p = 0; p < FT / 2; ++p) {
        typedef int i32x4 __attribute__((ext_vector_type(4)));
        if constexpr ((EPI & CG_EPI_MASKN) != 0) {
          // 16-byte chunk (8p + 2g + h) of row m (acc[2p + h]: features 32p + 8g + 4h .. + 3 of the
          // wave's 64) at chunk position (8p + 2g + h) ^ m of the row's 256 bytes: the 16 rows a
          // chunk column spans sit on distinct banks
          float* sE = reinterpret_cast<float*>(smem + NBUF * (STW + STX)) + wave * 1024;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *reinterpret_cast<f32x4*>(sE + m * 64 + (((8 * p + 2 * g + h) ^ m) << 2)) = acc[2 * p + h][j];
          if (p + 1 == FT / 2) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // lane l: feature l of each of the 16 rows, one 256-byte row piece per store
            const int f = nb * BN + 16 * FT * wf + lane;
            float bl = 0.f;
            if constexpr ((EPI & CG_EPI_BIAS) != 0) bl = f < N ? ep.bias[f] : 0.f;
            const uint32_t ecol = (uint32_t)(((rt & 63) * ldy + f) * 4);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float val = sE[r * 64 + (((lane >> 2) ^ r) << 2) + (lane & 3)] + bl;
              if (f < N)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, val), yres,
                                                      ecol + (uint32_t)(r * ldy * 4), 0, 0);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
          }
        } else if constexpr (sizeof(TO) == 2) {
          bf16x8 v;
          if constexpr ((EPI & CG_EPI_RES) != 0) {
            const bf16x8 r8 = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rres, rrow + 64 * p, 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = (bf16)(acc[2 * p][j][e] + (float)r8[e]);
              v[4 + e] = (bf16)(acc[2 * p + 1][j][e] + (float)r8[4 + e]);
            }
          } else if constexpr (NORM != MOC_NORM_NONE) {
            // features nb*BN + (BN/4) wf + 32 p + 8 g + e (acc[2p]) and + 4 + e (acc[2p+1])
            const float2 sr = sStat[rt + m];
            if constexpr (NORM == MOC_NORM_LAYERNORM) {
              const int f0 = nb * BN + 16 * FT * wf + 32 * p + 8 * g;
              const f32x4 u0 = *reinterpret_cast<const f32x4*>(nrm.u + f0);
              const f32x4 u1 = *reinterpret_cast<const f32x4*>(nrm.u + f0 + 4);
              const f32x4 v0 = *reinterpret_cast<const f32x4*>(nrm.v + f0);
              const f32x4 v1 = *reinterpret_cast<const f32x4*>(nrm.v + f0 + 4);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                v[e] = (bf16)(sr.y * (acc[2 * p][j][e] - sr.x * u0[e]) + v0[e]);
                v[4 + e] = (bf16)(sr.y * (acc[2 * p + 1][j][e] - sr.x * u1[e]) + v1[e]);
              }
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                v[e] = (bf16)(sr.y * acc[2 * p][j][e]);
                v[4 + e] = (bf16)(sr.y * acc[2 * p + 1][j][e]);
              }
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = (bf16)acc[2 * p][j][e];
              v[4 + e] = (bf16)acc[2 * p + 1][j][e];
            }
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), yres, vrow + 64 * p, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[2 * p][j]), yres, vrow + 128 * p, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[2 * p + 1][j]), yres,
                                                 vrow + 128 * p + 16, 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // Stage s computes from W(s) and X(s).  Per wave the loads go out as the batches W(p), X(p) of
  // stages 0 .. DEPTH-1, then one batch (of stage s + DEPTH, into the buffer stage s-1 used) at
  // each stage after its barrier.  A wave's loads complete in issue order, so with the batches
  // of stages s+1 .. s+DEPTH-1 allowed to stay in flight, "vmcnt <= (those batches) x kBatch"
  // means stage s's batch has landed.  After a tile's epilogue its stores are the newest
  // operations, so the next stage waits for everything instead.
#pragma unroll
  for (int p = 0; p < DEPTH; ++p)
    if (p < S) issue();
  // With one stage ahead, the wait for the next stage's loads is taken before a tile's epilogue
  // instead: the stage after it then needs no wait, and the stores are waited for one stage
  // later, when they have long completed.
  bool stored = false;
  for (int s = 0, kt = 0, t = lo + slot; s < S; ++s) {
    const int newer = min(DEPTH - 1, S - 1 - s);  // batches issued after stage s's
    if (DEPTH > 1) cg_wait_vm(stored ? 0 : newer * kBatch);
    else if (!stored) cg_wait_vm(0);
    __syncthreads();  // every wave's loads of stage s landed; every wave is done with stage s-1
    __builtin_amdgcn_sched_barrier(0);
    if (s + DEPTH < S) issue();
    __builtin_amdgcn_sched_barrier(0);
    compute(sW + (s % NBUF) * STW, sX + (s % NBUF) * STX);
    if constexpr (NORM != MOC_NORM_NONE) stats_stage(sX + (s % NBUF) * STX, kt == 0);
    stored = kt + 1 == nk;
    if (stored) {
      if constexpr (DEPTH == 1) cg_wait_vm(0);  // stage s + 1's loads (no stores outstanding)
      if constexpr (NORM != MOC_NORM_NONE) stats_finish(t);
      epilogue(t);
      t += nslot;
      kt = 0;
    } else {
      ++kt;
    }
  }
}

// Per-chapter sums of the dK|dV rows of chapters selected by several edges (csr order, fp32
// accumulation, rounded to bf16); chapters with one edge are read in place by the GEMM.  Every
// workgroup owns one 4 KB slice (256 threads x 16 bytes) of the 64-row chapter block and one of
// kMultiGroups shares of the chapters (u % kMultiGroups): it lists its share's chapters with
// several edges (the shared chapter, collisions) in LDS from one coalesced pass over csr_off, then
// sums its slice of each.
constexpr int kMultiGroups = 16;
__global__ __launch_bounds__(256) void dkv_multi_reduce_kernel(const bf16* __restrict__ dkv_edge,
                                                               const int32_t* __restrict__ n_uniq,
                                                               const int32_t* __restrict__ csr_off,
                                                               const int32_t* __restrict__ csr_edge, int64_t row_elems,
                                                               bf16* __restrict__ red) {
  __shared__ int list[1024];
  __shared__ int count;
  const int64_t nch = 64 * row_elems / 8;  // 16-byte chunks of one chapter block
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nu = n_uniq[0];
  for (int base = 0; base < nu; base += 1024) {
    if (threadIdx.x == 0) count = 0;
    __syncthreads();
    // this workgroup's share: chapters u with u % gridDim.y == blockIdx.y (the same set for every
    // slice, whatever order the list is built in)
    for (int u = base + threadIdx.x; u < min(nu, base + 1024); u += 256)
      if ((int)(u % gridDim.y) == (int)blockIdx.y && csr_off[u + 1] - csr_off[u] != 1) list[atomicAdd(&count, 1)] = u;
    __syncthreads();
    const int n = count;
    for (int k = 0; k < n && i < nch; ++k) {
      const int u = list[k];
      const int p0 = csr_off[u], p1 = csr_off[u + 1];
      float acc[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] = 0.f;
      for (int p = p0; p < p1; p += 4) {
        bf16x8 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (p + q < p1)
            v[q] = *reinterpret_cast<const bf16x8*>(dkv_edge + ((size_t)csr_edge[p + q] * 64 * row_elems + i * 8));
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (p + q < p1) {
#pragma unroll
            for (int x = 0; x < 8; ++x) acc[x] += (float)v[q][x];
          }
      }
      bf16x8 o;
#pragma unroll
      for (int x = 0; x < 8; ++x) o[x] = (bf16)acc[x];
      *reinterpret_cast<bf16x8*>(red + (size_t)u * 64 * row_elems + i * 8) = o;
    }
    __syncthreads();
  }
}

// The multi-edge chapters of a plan as a list (moc_common.h): one 1,024-thread workgroup, slots
// taken by an LDS counter, the count stored last.
__global__ __launch_bounds__(1024) void dkv_multi_list_kernel(const int32_t* __restrict__ n_uniq,
                                                              const int32_t* __restrict__ csr_off,
                                                              const int32_t* __restrict__ csr_edge, int64_t max_u,
                                                              int32_t* __restrict__ list) {
  __shared__ int count;
  if (threadIdx.x == 0) count = 0;
  __syncthreads();
  const int nu = (int)min((int64_t)n_uniq[0], max_u);
  for (int u = threadIdx.x; u < nu; u += 1024) {
    const int p0 = csr_off[u], cnt = csr_off[u + 1] - p0;
    if (cnt != 1) {
      int32_t* ent = list + 4 + kMultiEntry * atomicAdd(&count, 1);
      ent[0] = u;
      ent[1] = cnt;
      ent[2] = p0;
      ent[3] = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) ent[4 + i] = i < cnt ? csr_edge[p0 + i] : -1;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) list[0] = count;
}

// red[u] for the listed chapters: grid (16-byte slices of a chapter block / 256, groups); the
// workgroup of group y sums its slice of entries y, y + groups, ...  The count and the first
// entry are read together (one dependent load fewer than the scan of csr_off), each entry's rows
// in flight together, fp32 sums in edge order, one rounding.
__global__ __launch_bounds__(256) void dkv_multi_reduce_list_kernel(const bf16* __restrict__ dkv_edge,
                                                                    const int32_t* __restrict__ list, int64_t max_u,
                                                                    const int32_t* __restrict__ csr_edge,
                                                                    int64_t row_elems, bf16* __restrict__ red) {
  const int64_t nch = 64 * row_elems / 8;  // 16-byte chunks of one chapter block
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  for (int k = blockIdx.y; k < max_u; k += gridDim.y) {
    const i32x4* ent = reinterpret_cast<const i32x4*>(list + 4 + kMultiEntry * k);
    const i32x4 h = ent[0], e0 = ent[1], e1 = ent[2];
    if (k >= list[0]) break;
    if (i >= nch) continue;
    const int u = h[0], cnt = h[1], p0 = h[2];
    float acc[8];
#pragma unroll
    for (int x = 0; x < 8; ++x) acc[x] = 0.f;
    bf16x8 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int e = q < 4 ? e0[q] : e1[q - 4];
      if (q < cnt) v[q] = *reinterpret_cast<const bf16x8*>(dkv_edge + ((size_t)e * 64 * row_elems + i * 8));
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q < cnt) {
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[x] += (float)v[q][x];
      }
    for (int p = 8; p < cnt; ++p) {
      const bf16x8 w = *reinterpret_cast<const bf16x8*>(dkv_edge + ((size_t)csr_edge[p0 + p] * 64 * row_elems + i * 8));
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] += (float)w[x];
    }
    bf16x8 o;
#pragma unroll
    for (int x = 0; x < 8; ++x) o[x] = (bf16)acc[x];
    *reinterpret_cast<bf16x8*>(red + (size_t)u * 64 * row_elems + i * 8) = o;
  }
}

// [Wk; Wv] (rows kv of each, any of f32 / bf16) -> wkv [2 kv][d] bf16 and / or its transpose
// wkv_t [d][2 kv] (either may be null).  One workgroup per 64 x 64 tile: 16-byte loads, the tile
// kept in LDS as bf16 (rows padded to 72 elements), 16-byte stores of both layouts.  d and kv
// are multiples of 8 (host check).
template <typename TK, typename TV>
__global__ __launch_bounds__(256) void weight_pack_kernel(const TK* __restrict__ wk, const TV* __restrict__ wv,
                                                          int64_t nk, int64_t R, int64_t d, bf16* __restrict__ wkv,
                                                          bf16* __restrict__ wkv_t, int64_t ldt) {
  // rows r < nk from wk, nk <= r < R from wv; wkv [R][d], wkv_t [d][ldt] (columns R .. ldt-1 zero)
  __shared__ __attribute__((aligned(16))) bf16 tile[64][72];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int q = threadIdx.x + 256 * it, rr = q >> 3, cc = (q & 7) * 8;
    const int64_t r = r0 + rr, c = c0 + cc;
    bf16x8 v;
    if (r < R && c < d) {
      float f[8];
      if (r < nk) ChunkLoad8<TK>::run(wk + r * d + c, f);
      else ChunkLoad8<TV>::run(wv + (r - nk) * d + c, f);
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = (bf16)f[x];
      if (wkv) *reinterpret_cast<bf16x8*>(wkv + r * d + c) = v;
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = (bf16)0.f;
    }
    *reinterpret_cast<bf16x8*>(&tile[rr][cc]) = v;
  }
  if (!wkv_t) return;
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int q = threadIdx.x + 256 * it, cc = q >> 3, rr = (q & 7) * 8;
    const int64_t c = c0 + cc, r = r0 + rr;
    if (c >= d || r >= ldt) continue;
    bf16x8 v;
#pragma unroll
    for (int x = 0; x < 8; ++x) v[x] = tile[rr + x][cc];
    *reinterpret_cast<bf16x8*>(wkv_t + c * ldt + r) = v;
  }
}

// ------------------------------------------------------------ weight gradients
//   dW[n][k] = sum over 64-row blocks c < nblk and rows j < 64 of A_c[j][n] * B_c[j][k]
// A_c / B_c: the same per-block row sources as the GEMM above (a chapter's dK|dV rows, its bank
// rows, or rows 64c .. of a dense matrix, rows past the matrix end reading zero).  The output is
// small (N x K) and the reduction long, so the blocks are split over `splits` workgroups per
// 256 x 256 output tile, each writing an fp32 partial tile that cg_wgrad_reduce_kernel sums in a
// fixed order (deterministic).  Both operands keep the reduction index (rows) outermost, so the
// MFMA fragments (8 consecutive rows of one column per lane) come from gfx950's transposing LDS
// load ds_read_b64_tr_b16; the stage tiles are [64 rows][256 bf16] with 16-byte chunk c of row r
// at c ^ (2 (r & 3) | 8 ((r >> 3) & 3)).  A 16-lane group of one transposing load reads 4 rows x 2
// adjacent chunks and the two groups of a half-wave are 8 rows apart: the XOR puts those 16 chunks
// on 16 distinct 4-bank groups (XOR-ing by r & 3 instead had rows r and r ^ 1 share their chunk
// pair: 0.5 bank conflicts per access by the SQ counters, the kernel 2% slower).  Operands move
// global -> LDS by LDS DMA, one block ahead.
__device__ __forceinline__ int cg_tr_swz(int r) { return ((r & 3) << 1) | (((r >> 3) & 3) << 3); }
__device__ __forceinline__ int cg_tr_off(int row, int col) {
  return row * 512 + ((((col >> 3) ^ cg_tr_swz(row)) & 31) << 4) + ((col & 7) << 1);
}
typedef short cg_v4s __attribute__((ext_vector_type(4)));
// fragment: rows rb + 8 g + 0..7 (g = lane / 16) of column cb + lane % 16; within each 16-lane
// group, lane q supplies the address of row q / 4, columns 4 (q % 4) .. + 3
__device__ __forceinline__ bf16x8 cg_tr_frag(const char* base, int rb, int cb, int lane) {
  const int q = lane & 15;
  const int row = rb + 8 * (lane >> 4) + (q >> 2), col = cb + 4 * (q & 3);
  typedef __attribute__((address_space(3))) cg_v4s* lds_v4s;
  const cg_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + cg_tr_off(row, col)));
  const cg_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + cg_tr_off(row + 4, col)));
  const cg_v4s v[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8, v);
}

template <int SRC>
__device__ __forceinline__ uint32_t cg_block_bytes(int c, int64_t ld, int64_t rows) {
  if constexpr (SRC == CG_SRC_CONTIG) {
    const int64_t left = rows - (int64_t)c * 64;
    return (uint32_t)((left < 64 ? (left > 0 ? left : 0) : 64) * ld * 2);
  } else {
    return (uint32_t)(64 * ld * 2);
  }
}

template <int SRCA, int SRCB>
__global__ __launch_bounds__(kCgThreads) void chapter_wgrad_kernel(
    const bf16* __restrict__ a, const bf16* __restrict__ ared, int64_t lda, int64_t arows, const bf16* __restrict__ b,
    int64_t ldb, int64_t brows, const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq,
    const int32_t* __restrict__ csr_off, const int32_t* __restrict__ csr_edge, int64_t nblk_max, int N, int K,
    int splits, float* __restrict__ ws) {
  constexpr int STG = 64 * 512;  // one operand stage: 64 rows x 256 bf16
  __shared__ __attribute__((aligned(1024))) char smem[4 * STG];  // [buf][A | B]
  const int nkb = K >> 8, tiles = (N >> 8) * nkb;
  const int64_t t = xcd_tile((int64_t)tiles * splits);  // split major: a split's tiles share an XCD
  if (t < 0) return;
  const int tile = (int)(t % tiles), split = (int)(t / tiles);
  const int n0 = (tile / nkb) * 256, k0 = (tile % nkb) * 256;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = rfl(tid >> 6);
  const int wn = wave >> 2, wk = wave & 3;  // wave tile: 128 (n) x 64 (k)
  const int nblk = n_uniq ? rfl((int)min((int64_t)n_uniq[0], nblk_max)) : (int)nblk_max;
  const int per = (nblk + splits - 1) / splits;
  const int s0 = min(nblk, split * per), s1 = min(nblk, s0 + per);

  // DMA: instruction i of wave w fills LDS rows 16 i + 2 w + lane / 32, physical chunk lane % 32
  const int r0 = 2 * wave + (lane >> 5);
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (lane & 31) ^ cg_tr_swz(16 * i + r0);
    aoff[i] = (uint32_t)(((int64_t)(16 * i + r0) * lda + n0 + 8 * c) * 2);
    boff[i] = (uint32_t)(((int64_t)(16 * i + r0) * ldb + k0 + 8 * c) * 2);
  }
  auto issue = [&](int blk, int buf) {
    const bf16* ab = cg_src_rows<SRCA>(blk, a, ared, lda, uniq, csr_off, csr_edge);
    const bf16* bb = cg_src_rows<SRCB>(blk, b, nullptr, ldb, uniq, csr_off, csr_edge);
    const __amdgpu_buffer_rsrc_t ar = CG_RSRC(ab, cg_block_bytes<SRCA>(blk, lda, arows));
    const __amdgpu_buffer_rsrc_t br = CG_RSRC(bb, cg_block_bytes<SRCB>(blk, ldb, brows));
    const char* da = smem + buf * 2 * STG + wave * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cg_dma16(ar, aoff[i], 0u, da + 8192 * i);
      cg_dma16(br, boff[i], 0u, da + STG + 8192 * i);
    }
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (s0 < s1) issue(s0, 0);
  for (int st = s0; st < s1; ++st) {
    const int buf = (st - s0) & 1;
    cg_wait_vm(0);
    __syncthreads();  // block st landed for every wave; every wave is done with block st-1
    __builtin_amdgcn_sched_barrier(0);
    if (st + 1 < s1) issue(st + 1, buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    const char* As = smem + buf * 2 * STG;
    const char* Bs = As + STG;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 bfr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = cg_tr_frag(Bs, 32 * ks, 64 * wk + 16 * j, lane);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bf16x8 afr = cg_tr_frag(As, 32 * ks, 128 * wn + 16 * i, lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) mma(acc[i][j], afr, bfr[j]);
      }
    }
  }
  // partial tile in accumulator order: [split][tile][wave][i][j][lane] f32x4
  f32x4* out = reinterpret_cast<f32x4*>(ws) + (((size_t)split * tiles + tile) * 8 + wave) * 32 * 64 + lane;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) out[(i * 4 + j) * 64] = acc[i][j];
}

// dW[n, k] = sum over splits (in order) of the partial tiles; one thread per f32x4.
template <typename TO>
__global__ __launch_bounds__(256) void cg_wgrad_reduce_kernel(const float* __restrict__ ws, int splits, int tiles,
                                                              int nkb, int K, TO* __restrict__ dw) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;  // f32x4 index within one split
  const int64_t per_split = (int64_t)tiles * 8 * 32 * 64;
  if (p >= per_split) return;
  f32x4 s = reinterpret_cast<const f32x4*>(ws)[p];
  for (int sp = 1; sp < splits; ++sp) s += reinterpret_cast<const f32x4*>(ws)[sp * per_split + p];
  const int lane = (int)(p & 63), ij = (int)((p >> 6) & 31), wave = (int)((p >> 11) & 7);
  const int tile = (int)(p >> 14);
  const int i = ij >> 2, j = ij & 3, wn = wave >> 2, wk = wave & 3;
  const int n = (tile / nkb) * 256 + 128 * wn + 16 * i + 4 * (lane >> 4);
  const int64_t k = (int64_t)(tile % nkb) * 256 + 64 * wk + 16 * j + (lane & 15);
#pragma unroll
  for (int e = 0; e < 4; ++e) dw[(int64_t)(n + e) * K + k] = from_f<TO>(s[e]);
}

// W~ = W diag(gamma) (bf16, rounded once), u[n] = sum_k W~[n][k] (over the rounded values the GEMM
// multiplies), v[n] = sum_k W[n][k] beta[k]; one wave per output row, lane-strided sums reduced
// in a fixed order
__global__ __launch_bounds__(256) void norm_fold_kernel(const bf16* __restrict__ w, int N, int K,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, bf16* __restrict__ w_out,
                                                        float* __restrict__ u, float* __restrict__ v) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;
  const bf16* wr = w + (int64_t)n * K;
  bf16* wo = w_out + (int64_t)n * K;
  float su = 0.f, sv = 0.f;
  for (int k0 = 8 * lane; k0 < K; k0 += 512) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(wr + k0);
    const f32x4 g0 = *reinterpret_cast<const f32x4*>(gamma + k0), g1 = *reinterpret_cast<const f32x4*>(gamma + k0 + 4);
    f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (beta) {
      b0 = *reinterpret_cast<const f32x4*>(beta + k0);
      b1 = *reinterpret_cast<const f32x4*>(beta + k0 + 4);
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float wf = (float)a[e];
      o[e] = (bf16)(wf * (e < 4 ? g0[e] : g1[e - 4]));
      su += (float)o[e];
      sv += wf * (e < 4 ? b0[e] : b1[e - 4]);
    }
    *reinterpret_cast<bf16x8*>(wo + k0) = o;
  }
  if (u) {
    su = wave_sum(su);
    sv = wave_sum(sv);
    if (lane == 0) {
      u[n] = su;
      if (v) v[n] = sv;
    }
  }
}

int cg_grid() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return (cus + 7) / 8 * 8;
}

int cg_check(const char* who, int64_t ldx, int N, int K, int64_t max_u, int64_t ldy) {
  MOC_REQUIRE(N > 0 && N % 256 == 0, MOC_ERR_UNSUPPORTED, "%s: N=%d must be a positive multiple of 256", who, N);
  MOC_REQUIRE(K > 0 && K % 64 == 0, MOC_ERR_UNSUPPORTED, "%s: K=%d must be a positive multiple of 64", who, K);
  MOC_REQUIRE(ldx >= K && ldx % 8 == 0, MOC_ERR_ARG, "%s: row stride %lld (K=%d)", who, (long long)ldx, K);
  MOC_REQUIRE(ldy >= N && ldy % 8 == 0, MOC_ERR_ARG, "%s: output row stride %lld (N=%d)", who, (long long)ldy, N);
  MOC_REQUIRE(64 * ldx * 2 < ((int64_t)1 << 31) && 64 * ldy * 4 < ((int64_t)1 << 31) &&
                  (int64_t)384 * K * 2 < ((int64_t)1 << 31) && max_u < ((int64_t)1 << 30),
              MOC_ERR_UNSUPPORTED, "%s: problem too large", who);
  return MOC_OK;
}

// workgroups per output tile of the weight gradients: fill `budget` CUs (256: the chip), but give
// each at least 8 row blocks
int cg_wgrad_splits(int tiles, int64_t blocks, int budget = 256) {
  int64_t s = budget / tiles;
  const int64_t by_len = (blocks + 7) / 8;
  if (s > by_len) s = by_len;
  if (s < 1) s = 1;
  return (int)s;
}

int cg_wgrad_reduce(void* ws, int splits, int tiles, int K, int out_dtype, void* dw, hipStream_t stream) {
  const int64_t n4 = (int64_t)tiles * 8 * 32 * 64;
  const dim3 rgrid((unsigned)((n4 + 255) / 256));
  if (out_dtype == MOC_F32)
    hipLaunchKernelGGL(cg_wgrad_reduce_kernel<float>, rgrid, dim3(256), 0, stream, (const float*)ws, splits, tiles,
                       K / 256, K, (float*)dw);
  else
    hipLaunchKernelGGL(cg_wgrad_reduce_kernel<bf16>, rgrid, dim3(256), 0, stream, (const float*)ws, splits, tiles,
                       K / 256, K, (bf16*)dw);
  return check_launch("cg_wgrad_reduce_kernel");
}

}  // namespace

// Dense weight gradient dw [N][K] = dy^T x over R rows (dy [R][N], x [R][K], both bf16, row
// strides N and K) on the chapter weight-gradient kernel; used by moc_linear_wgrad for the
// shapes it tiles (N, K multiples of 256).  The split count (and so the workspace) follows the
// same rule as moc_linear_wgrad_workspace.
int chapter_wgrad_dense(const void* dy, const void* x, int64_t R, int64_t N, int64_t K, void* ws, int out_dtype,
                        void* dw, hipStream_t stream) {
  const int tiles = (int)((N / 256) * (K / 256));
  const int64_t blocks = (R + 63) / 64;
  const int splits = cg_wgrad_splits(tiles, blocks);
  const dim3 grid(xcd_grid((int64_t)tiles * splits));
  hipLaunchKernelGGL((chapter_wgrad_kernel<CG_SRC_CONTIG, CG_SRC_CONTIG>), grid, dim3(kCgThreads), 0, stream,
                     (const bf16*)dy, (const bf16*)nullptr, (int64_t)N, R, (const bf16*)x, (int64_t)K, R, nullptr,
                     nullptr, nullptr, nullptr, blocks, (int)N, (int)K, splits, (float*)ws);
  if (int rc = check_launch("chapter_wgrad_kernel(dense)")) return rc;
  return cg_wgrad_reduce(ws, splits, tiles, (int)K, out_dtype, dw, stream);
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_chapter_project(const void* rows, int64_t ld, int gather, const int32_t* uniq, const int32_t* n_uniq,
                        int64_t max_u, const void* w, int N, int K, void* y, int64_t ldy, hipStream_t stream) {
  MOC_REQUIRE(rows && n_uniq && w && y && (uniq || !gather), MOC_ERR_ARG, "moc_chapter_project: null pointer");
  MOC_REQUIRE(max_u >= 0, MOC_ERR_ARG, "moc_chapter_project: max_u %lld", (long long)max_u);
  if (int rc = cg_check("moc_chapter_project", ld, N, K, max_u, ldy)) return rc;
  if (max_u == 0) return MOC_OK;
  const dim3 grid((unsigned)cg_grid());
#define MOC_CGP(SRC, BN)                                                                                            \
  hipLaunchKernelGGL((chapter_gemm_kernel<SRC, CG_DST_CONTIG, bf16, 256, kCgDepth256, MOC_NORM_NONE, BN>), grid,       \
                     dim3(kCgThreads), 0, stream, (const bf16*)rows, nullptr, ld, uniq, n_uniq, nullptr, nullptr,    \
                     max_u, (const bf16*)w, N, K, (bf16*)y, ldy, max_u * 64, max_u * 64, CgNorm{})
  const bool wide = N % 384 == 0;
  if (gather) {
    if (wide) MOC_CGP(CG_SRC_GATHER, 384); else MOC_CGP(CG_SRC_GATHER, 256);
  } else {
    if (wide) MOC_CGP(CG_SRC_CONTIG, 384); else MOC_CGP(CG_SRC_CONTIG, 256);
  }
#undef MOC_CGP
  return check_launch("chapter_gemm_kernel(project)");
}

int moc_chapter_dx(const void* dkv_edge, int64_t ld, const int32_t* uniq, const int32_t* n_uniq, int64_t max_u,
                   const int32_t* csr_off, const int32_t* csr_edge, void* red, const void* w_t, int N, int K,
                   int out_dtype, void* out, int64_t ldo, int out_bank_rows, hipStream_t stream) {
  MOC_REQUIRE(dkv_edge && uniq && n_uniq && csr_off && csr_edge && red && w_t && out, MOC_ERR_ARG,
              "moc_chapter_dx: null pointer");
  MOC_REQUIRE(max_u >= 0, MOC_ERR_ARG, "moc_chapter_dx: max_u %lld", (long long)max_u);
  MOC_REQUIRE(out_dtype == MOC_BF16 || out_dtype == MOC_F32, MOC_ERR_UNSUPPORTED, "moc_chapter_dx: out dtype %d",
              out_dtype);
  if (int rc = cg_check("moc_chapter_dx", ld, N, K, max_u, ldo)) return rc;
  if (max_u == 0) return MOC_OK;
  const dim3 grid((unsigned)cg_grid());
  // 256 x 384 tiles where N allows (one stage ahead, 2 x 80 KB of LDS: a sixth less operand
  // traffic per product than 256 x 256; c3 dX 102 -> 76 us), else 128 x 256 tiles two stages ahead
#define MOC_CGDX(DST, TO)                                                                                           \
  if (N % 384 == 0)                                                                                                 \
    hipLaunchKernelGGL((chapter_gemm_kernel<CG_SRC_EDGE, DST, TO, 256, kCgDepth256, MOC_NORM_NONE, 384>), grid,      \
                       dim3(kCgThreads), 0, stream, (const bf16*)dkv_edge, (const bf16*)red, ld, uniq, n_uniq,       \
                       csr_off, csr_edge, max_u, (const bf16*)w_t, N, K, (TO*)out, ldo, max_u * 64, max_u * 64,     \
                       CgNorm{});                                                                                   \
  else                                                                                                              \
    hipLaunchKernelGGL((chapter_gemm_kernel<CG_SRC_EDGE, DST, TO, kCgDxRows, kCgDepth128>), grid, dim3(kCgThreads), \
                       0, stream, (const bf16*)dkv_edge, (const bf16*)red, ld, uniq, n_uniq, csr_off, csr_edge,     \
                       max_u, (const bf16*)w_t, N, K, (TO*)out, ldo, max_u * 64, max_u * 64, CgNorm{})
  if (out_bank_rows) {
    if (out_dtype == MOC_BF16) MOC_CGDX(CG_DST_BANK, bf16); else MOC_CGDX(CG_DST_BANK, float);
  } else {
    if (out_dtype == MOC_BF16) MOC_CGDX(CG_DST_CONTIG, bf16); else MOC_CGDX(CG_DST_CONTIG, float);
  }
#undef MOC_CGDX
  return check_launch("chapter_gemm_kernel(dx)");
}

}  // extern "C"

namespace moc {
namespace {

// y [R][N] = x [R][K] w^T (+ epilogue options) over contiguous rows.  Tiles: 128 x 256 two
// k-stages ahead while the 256 x 384 (or 256 x 256) tiles would not fill two rounds of the
// persistent grid (the c3 q / o projections: 192 tiles against 64), else the wide tiles one
// stage ahead (the bank-sized products of the token path: thousands of tiles, a sixth to a third
// less operand traffic per product).
template <typename TO, int EPI>
int rows_gemm(const char* who, const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, void* y,
              int64_t ldy, CgEpi ep, hipStream_t stream) {
  const int64_t blocks = (R + 63) / 64;
  if (R == 0) return MOC_OK;
  const int grid = cg_grid();
  const bool n384 = (EPI & CG_EPI_MASKN) == 0 && N % 384 == 0;
  const int64_t wide_tiles = (R + 255) / 256 * ((N + (n384 ? 383 : 255)) / (n384 ? 384 : 256));
  // (the any-N epilogue's LDS staging leaves room for one k-stage ahead only)
  constexpr int kNarrowDepth = (EPI & CG_EPI_MASKN) ? 1 : kCgDepth128;
#define MOC_RG(BM, DEPTH, BN)                                                                                     \
  hipLaunchKernelGGL((chapter_gemm_kernel<CG_SRC_CONTIG, CG_DST_CONTIG, TO, BM, DEPTH, MOC_NORM_NONE, BN, EPI>),  \
                     dim3((unsigned)grid), dim3(kCgThreads), 0, stream, (const bf16*)x, nullptr, ldx, nullptr,    \
                     nullptr, nullptr, nullptr, blocks, (const bf16*)w, N, K, (TO*)y, ldy, R, R, CgNorm{}, ep)
  if (wide_tiles < 2 * (int64_t)grid) {
    MOC_RG(128, kNarrowDepth, 256);
  } else if constexpr ((EPI & CG_EPI_MASKN) == 0) {
    if (n384) MOC_RG(256, kCgDepth256, 384);
    else MOC_RG(256, kCgDepth256, 256);
  } else {
    MOC_RG(256, kCgDepth256, 256);
  }
#undef MOC_RG
  return check_launch(who);
}

}  // namespace
}  // namespace moc

extern "C" {

int moc_rows_linear(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, void* y, int64_t ldy,
                    hipStream_t stream) {
  MOC_REQUIRE(x && w && y, MOC_ERR_ARG, "moc_rows_linear: null pointer");
  MOC_REQUIRE(R >= 0 && R < ((int64_t)1 << 36), MOC_ERR_ARG, "moc_rows_linear: R=%lld", (long long)R);
  if (int rc = cg_check("moc_rows_linear", ldx, N, K, (R + 63) / 64, ldy)) return rc;
  return rows_gemm<bf16, 0>("chapter_gemm_kernel(rows)", x, ldx, R, w, N, K, y, ldy, CgEpi{}, stream);
}

int moc_rows_linear_residual(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, const void* res,
                             int64_t ldr, void* y, int64_t ldy, hipStream_t stream) {
  MOC_REQUIRE(x && w && res && y, MOC_ERR_ARG, "moc_rows_linear_residual: null pointer");
  MOC_REQUIRE(R >= 0 && R < ((int64_t)1 << 36), MOC_ERR_ARG, "moc_rows_linear_residual: R=%lld", (long long)R);
  MOC_REQUIRE(ldr >= N && ldr % 8 == 0 && 64 * ldr * 2 < ((int64_t)1 << 31) && ((uintptr_t)res & 15) == 0,
              MOC_ERR_ARG, "moc_rows_linear_residual: residual row stride %lld (N=%d), 16-byte aligned rows",
              (long long)ldr, N);
  if (int rc = cg_check("moc_rows_linear_residual", ldx, N, K, (R + 63) / 64, ldy)) return rc;
  return rows_gemm<bf16, CG_EPI_RES>("chapter_gemm_kernel(rows, residual)", x, ldx, R, w, N, K, y, ldy,
                                     CgEpi{(const bf16*)res, ldr, nullptr}, stream);
}

int moc_rows_linear_f32(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, const float* bias,
                        float* y, int64_t ldy, hipStream_t stream) {
  MOC_REQUIRE(x && w && y, MOC_ERR_ARG, "moc_rows_linear_f32: null pointer");
  MOC_REQUIRE(R >= 0 && R < ((int64_t)1 << 36), MOC_ERR_ARG, "moc_rows_linear_f32: R=%lld", (long long)R);
  MOC_REQUIRE(N > 0 && K > 0 && K % 64 == 0, MOC_ERR_UNSUPPORTED, "moc_rows_linear_f32: N=%d, K=%d (K a multiple of 64)",
              N, K);
  MOC_REQUIRE(ldx >= K && ldx % 8 == 0 && ldy >= N && 64 * ldx * 2 < ((int64_t)1 << 31) &&
                  64 * ldy * 4 < ((int64_t)1 << 31) && (int64_t)256 * K * 2 < ((int64_t)1 << 31),
              MOC_ERR_ARG, "moc_rows_linear_f32: row strides %lld, %lld (N=%d, K=%d)", (long long)ldx, (long long)ldy,
              N, K);
  const CgEpi ep{nullptr, 0, bias};
  if (bias)
    return rows_gemm<float, CG_EPI_MASKN | CG_EPI_BIAS>("chapter_gemm_kernel(rows, f32, bias)", x, ldx, R, w, N, K,
                                                        y, ldy, ep, stream);
  return rows_gemm<float, CG_EPI_MASKN>("chapter_gemm_kernel(rows, f32)", x, ldx, R, w, N, K, y, ldy, ep, stream);
}

int moc_norm_fold_weight(const void* w, int N, int K, const float* gamma, const float* beta, void* w_out, float* u,
                         float* v, hipStream_t stream) {
  MOC_REQUIRE(w && gamma && w_out, MOC_ERR_ARG, "moc_norm_fold_weight: null pointer");
  MOC_REQUIRE(N > 0 && K > 0 && K % 8 == 0, MOC_ERR_ARG, "moc_norm_fold_weight: N=%d K=%d (K a multiple of 8)", N, K);
  MOC_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)w_out & 15) == 0 && ((uintptr_t)gamma & 15) == 0 &&
                  ((uintptr_t)beta & 15) == 0,
              MOC_ERR_ARG, "moc_norm_fold_weight: w, w_out, gamma and beta must be 16-byte aligned");
  MOC_REQUIRE(!beta || (u && v), MOC_ERR_ARG, "moc_norm_fold_weight: a bias needs u and v");
  MOC_REQUIRE(!v || u, MOC_ERR_ARG, "moc_norm_fold_weight: v needs u");
  hipLaunchKernelGGL(norm_fold_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, (const bf16*)w, N, K,
                     gamma, beta, (bf16*)w_out, u, v);
  return check_launch("norm_fold_kernel");
}

int moc_rows_linear_norm(const void* x, int64_t ldx, int64_t R, const void* w_folded, int N, int K, int norm,
                         float eps, const float* u, const float* v, void* y, int64_t ldy, float* mean_out,
                         float* rstd_out, hipStream_t stream) {
  MOC_REQUIRE(x && w_folded && y, MOC_ERR_ARG, "moc_rows_linear_norm: null pointer");
  MOC_REQUIRE(norm == MOC_NORM_RMS || norm == MOC_NORM_LAYERNORM, MOC_ERR_ARG, "moc_rows_linear_norm: norm %d",
              norm);
  MOC_REQUIRE(norm == MOC_NORM_RMS || (u && v && ((uintptr_t)u & 15) == 0 && ((uintptr_t)v & 15) == 0), MOC_ERR_ARG,
              "moc_rows_linear_norm: LayerNorm needs 16-byte aligned u and v");
  MOC_REQUIRE(R >= 0 && R < ((int64_t)1 << 36) && eps >= 0.f, MOC_ERR_ARG, "moc_rows_linear_norm: R=%lld eps=%g",
              (long long)R, (double)eps);
  const int64_t blocks = (R + 63) / 64;
  if (int rc = cg_check("moc_rows_linear_norm", ldx, N, K, blocks, ldy)) return rc;
  if (R == 0) return MOC_OK;
  const CgNorm nrm{eps, u, v, mean_out, rstd_out};
  if (norm == MOC_NORM_RMS)
    hipLaunchKernelGGL((chapter_gemm_kernel<CG_SRC_CONTIG, CG_DST_CONTIG, bf16, 128, kCgDepth128, MOC_NORM_RMS>),
                       dim3((unsigned)cg_grid()), dim3(kCgThreads), 0, stream, (const bf16*)x, nullptr, ldx, nullptr,
                       nullptr, nullptr, nullptr, blocks, (const bf16*)w_folded, N, K, (bf16*)y, ldy, R, R, nrm);
  else
    hipLaunchKernelGGL((chapter_gemm_kernel<CG_SRC_CONTIG, CG_DST_CONTIG, bf16, 128, kCgDepth128, MOC_NORM_LAYERNORM>),
                       dim3((unsigned)cg_grid()), dim3(kCgThreads), 0, stream, (const bf16*)x, nullptr, ldx, nullptr,
                       nullptr, nullptr, nullptr, blocks, (const bf16*)w_folded, N, K, (bf16*)y, ldy, R, R, nrm);
  return check_launch("chapter_gemm_kernel(rows, norm)");
}

int moc_dkv_multi_reduce(const void* dkv_edge, int64_t ld, const int32_t* n_uniq, int64_t max_u,
                         const int32_t* csr_off, const int32_t* csr_edge, void* red, hipStream_t stream) {
  MOC_REQUIRE(dkv_edge && n_uniq && csr_off && csr_edge && red, MOC_ERR_ARG, "moc_dkv_multi_reduce: null pointer");
  MOC_REQUIRE(ld > 0 && ld % 8 == 0 && max_u >= 0, MOC_ERR_ARG, "moc_dkv_multi_reduce: ld=%lld", (long long)ld);
  if (max_u == 0) return MOC_OK;
  hipLaunchKernelGGL(dkv_multi_reduce_kernel, dim3((unsigned)((64 * ld / 8 + 255) / 256), kMultiGroups), dim3(256), 0,
                     stream, (const bf16*)dkv_edge, n_uniq, csr_off, csr_edge, ld, (bf16*)red);
  return check_launch("dkv_multi_reduce_kernel");
}

size_t moc_chapter_wgrad_workspace(int N, int K, int64_t max_u) {
  if (N <= 0 || K <= 0 || N % 256 || K % 256) return 0;
  const int tiles = (N / 256) * (K / 256);
  return (size_t)cg_wgrad_splits(tiles, max_u) * tiles * 256 * 256 * sizeof(float);
}

int moc_chapter_wgrad(const void* dkv_edge, int64_t lda, const void* red, const void* x, int64_t ldx, int gather,
                      const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                      const int32_t* csr_edge, int N, int K, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                      hipStream_t stream) {
  return chapter_wgrad_budget(dkv_edge, lda, red, x, ldx, gather, uniq, n_uniq, max_u, csr_off, csr_edge, N, K, ws,
                              ws_bytes, out_dtype, dw, 256, stream);
}

}  // extern "C"

namespace moc {

int dkv_multi_list(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                   int32_t* list, hipStream_t stream) {
  MOC_REQUIRE(n_uniq && csr_off && csr_edge && list && ((uintptr_t)list & 15) == 0 && max_u >= 0, MOC_ERR_ARG,
              "dkv_multi_list: null or unaligned pointer");
  hipLaunchKernelGGL(dkv_multi_list_kernel, dim3(1), dim3(1024), 0, stream, n_uniq, csr_off, csr_edge, max_u, list);
  return check_launch("dkv_multi_list_kernel");
}

int dkv_multi_reduce_list(const void* dkv_edge, int64_t ld, const int32_t* list, int64_t max_u,
                          const int32_t* csr_edge, void* red, hipStream_t stream) {
  MOC_REQUIRE(dkv_edge && list && csr_edge && red && ((uintptr_t)list & 15) == 0, MOC_ERR_ARG,
              "dkv_multi_reduce_list: null or unaligned pointer");
  MOC_REQUIRE(ld > 0 && ld % 8 == 0 && max_u >= 0, MOC_ERR_ARG, "dkv_multi_reduce_list: ld=%lld", (long long)ld);
  if (max_u == 0) return MOC_OK;
  hipLaunchKernelGGL(dkv_multi_reduce_list_kernel, dim3((unsigned)((64 * ld / 8 + 255) / 256), kMultiGroups), dim3(256),
                     0, stream, (const bf16*)dkv_edge, list, max_u, csr_edge, ld, (bf16*)red);
  return check_launch("dkv_multi_reduce_list_kernel");
}

int chapter_wgrad_budget(const void* dkv_edge, int64_t lda, const void* red, const void* x, int64_t ldx, int gather,
                         const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                         const int32_t* csr_edge, int N, int K, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                         int budget, hipStream_t stream) {
  MOC_REQUIRE(dkv_edge && red && x && uniq && n_uniq && csr_off && csr_edge && ws && dw, MOC_ERR_ARG,
              "moc_chapter_wgrad: null pointer");
  MOC_REQUIRE(N > 0 && N % 256 == 0 && K > 0 && K % 256 == 0, MOC_ERR_UNSUPPORTED,
              "moc_chapter_wgrad: N=%d, K=%d must be positive multiples of 256", N, K);
  MOC_REQUIRE(lda >= N && lda % 8 == 0 && ldx >= K && ldx % 8 == 0 && 64 * lda * 2 < ((int64_t)1 << 31) &&
                  64 * ldx * 2 < ((int64_t)1 << 31) && max_u >= 0 && max_u < ((int64_t)1 << 30),
              MOC_ERR_ARG, "moc_chapter_wgrad: bad strides");
  MOC_REQUIRE(ws_bytes >= moc_chapter_wgrad_workspace(N, K, max_u), MOC_ERR_ARG, "moc_chapter_wgrad: workspace too small");
  MOC_REQUIRE(out_dtype == MOC_F32 || out_dtype == MOC_BF16, MOC_ERR_UNSUPPORTED, "moc_chapter_wgrad: out dtype %d",
              out_dtype);
  MOC_REQUIRE(budget > 0 && budget <= 256, MOC_ERR_ARG, "chapter weight gradient: workgroup budget %d", budget);
  const int tiles = (N / 256) * (K / 256), splits = cg_wgrad_splits(tiles, max_u, budget);
  const dim3 grid(xcd_grid((int64_t)tiles * splits));
  if (gather)
    hipLaunchKernelGGL((chapter_wgrad_kernel<CG_SRC_EDGE, CG_SRC_GATHER>), grid, dim3(kCgThreads), 0, stream,
                       (const bf16*)dkv_edge, (const bf16*)red, lda, (int64_t)0, (const bf16*)x, ldx, (int64_t)0, uniq,
                       n_uniq, csr_off, csr_edge, max_u, N, K, splits, (float*)ws);
  else
    hipLaunchKernelGGL((chapter_wgrad_kernel<CG_SRC_EDGE, CG_SRC_CONTIG>), grid, dim3(kCgThreads), 0, stream,
                       (const bf16*)dkv_edge, (const bf16*)red, lda, (int64_t)0, (const bf16*)x, ldx, max_u * 64, uniq,
                       n_uniq, csr_off, csr_edge, max_u, N, K, splits, (float*)ws);
  if (int rc = check_launch("chapter_wgrad_kernel")) return rc;
  return cg_wgrad_reduce(ws, splits, tiles, K, out_dtype, dw, stream);
}

}  // namespace moc

extern "C" {

int moc_weight_pack(const void* wk, int wk_dtype, const void* wv, int wv_dtype, int64_t kv, int64_t d, void* wkv,
                    void* wkv_t, hipStream_t stream) {
  MOC_REQUIRE(wk && wv && (wkv || wkv_t), MOC_ERR_ARG, "moc_weight_pack: null pointer");
  MOC_REQUIRE(kv > 0 && d > 0 && kv % 8 == 0 && d % 8 == 0 && 2 * kv * d < ((int64_t)1 << 40), MOC_ERR_ARG,
              "moc_weight_pack: kv=%lld, d=%lld must be positive multiples of 8", (long long)kv, (long long)d);
  const dim3 grid((unsigned)((d + 63) / 64), (unsigned)((2 * kv + 63) / 64));
#define MOC_WP(TK, TV)                                                                                           \
  hipLaunchKernelGGL((weight_pack_kernel<TK, TV>), grid, dim3(256), 0, stream, (const TK*)wk, (const TV*)wv, kv, \
                     2 * kv, d, (bf16*)wkv, (bf16*)wkv_t, 2 * kv)
  if (wk_dtype == MOC_BF16 && wv_dtype == MOC_BF16) MOC_WP(bf16, bf16);
  else if (wk_dtype == MOC_F32 && wv_dtype == MOC_F32) MOC_WP(float, float);
  else if (wk_dtype == MOC_BF16 && wv_dtype == MOC_F32) MOC_WP(bf16, float);
  else if (wk_dtype == MOC_F32 && wv_dtype == MOC_BF16) MOC_WP(float, bf16);
  else return set_error(MOC_ERR_UNSUPPORTED, "moc_weight_pack: dtypes %d, %d", wk_dtype, wv_dtype);
#undef MOC_WP
  return check_launch("weight_pack_kernel");
}

int moc_weight_transpose(const void* w, int w_dtype, int64_t N, int64_t K, void* wt, int64_t ldt,
                         hipStream_t stream) {
  MOC_REQUIRE(w && wt, MOC_ERR_ARG, "moc_weight_transpose: null pointer");
  MOC_REQUIRE(N > 0 && K > 0 && K % 8 == 0 && ldt >= N && ldt % 8 == 0 && ldt * K < ((int64_t)1 << 40), MOC_ERR_ARG,
              "moc_weight_transpose: N=%lld, K=%lld (a multiple of 8), ldt=%lld (>= N, a multiple of 8)",
              (long long)N, (long long)K, (long long)ldt);
  MOC_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)wt & 15) == 0, MOC_ERR_ARG,
              "moc_weight_transpose: w and wt must be 16-byte aligned");
  const dim3 grid((unsigned)((K + 63) / 64), (unsigned)((ldt + 63) / 64));
  if (w_dtype == MOC_BF16)
    hipLaunchKernelGGL((weight_pack_kernel<bf16, bf16>), grid, dim3(256), 0, stream, (const bf16*)w, (const bf16*)w, N,
                       N, K, (bf16*)nullptr, (bf16*)wt, ldt);
  else if (w_dtype == MOC_F32)
    hipLaunchKernelGGL((weight_pack_kernel<float, float>), grid, dim3(256), 0, stream, (const float*)w,
                       (const float*)w, N, N, K, (bf16*)nullptr, (bf16*)wt, ldt);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_weight_transpose: dtype %d", w_dtype);
  return check_launch("weight_pack_kernel");
}

}  // extern "C"
