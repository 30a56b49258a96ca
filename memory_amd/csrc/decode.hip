// Single-token decode over precomputed per-layer K / V chapter tiles.
//
// Step of the sequence-routed memory layer with L = 1 (the decode use of
// memory_transformer/model.py:612-692 -> memory_attention.py:458-478) when the
// chapters and their weights omega are fixed for the generation: K / V of every
// chapter are precomputed once per layer (kv_project over all chapters), so a step
// only reads the selected tiles.  HBM-bound: each distinct (chapter, kv head) tile
// is read once per step however many sequences selected it (chapter plan over the
// (sequence, slot) edges).
//
// The omega-weighted memory rows of the reference (memory = memory * omega before the
// K/V projection) give K = omega K_c and V = omega V_c, so per edge (b, slot) and query
// head: s_j = omega * scale * q . k_j, o = omega * sum_j p_j v_j / sum_j p_j and
// lse = log2 sum_j 2^(s_j log2 e): exactly the chapter-centric partial attention of the
// token-routed path with a per-edge logit and output factor (sparse_fwd_launch: one
// wave per (chapter, kv head) unit, K fragments from HBM, V^T through transposing LDS
// reads).  moc_sparse_combine (joint mode, rpe = H) merges the slots of a sequence.  The plan is
// fixed for a whole generation, so the first 16 edges of every chapter are tabulated once
// (moc_decode_row_table): a unit then requests its rows' edge ids together with its plan entries
// instead of after them, and its q rows go out together with its K / V tiles.
#include "moc_common.h"

using namespace moc;

namespace {

// row_tab[u * W + j] = the j-th edge (csr order) of distinct chapter u, -1 past its edges or past
// n_uniq; one thread per entry.
__global__ __launch_bounds__(256) void decode_row_table_kernel(const int32_t* __restrict__ n_uniq,
                                                               const int32_t* __restrict__ csr_off,
                                                               const int32_t* __restrict__ csr_edge, int64_t max_u,
                                                               int W, int32_t* __restrict__ row_tab) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t u = i / W;
  const int j = (int)(i % W);
  if (u >= max_u) return;
  int32_t e = -1;
  if (u < n_uniq[0]) {
    const int32_t p0 = csr_off[u], cnt = csr_off[u + 1] - p0;
    if (j < cnt) e = csr_edge[p0 + j];
  }
  row_tab[i] = e;
}

}  // namespace

extern "C" {

int moc_plan_row_table(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                       int width, int32_t* row_tab, hipStream_t stream) {
  MOC_REQUIRE(n_uniq && csr_off && csr_edge && row_tab, MOC_ERR_ARG, "moc_plan_row_table: null pointer");
  MOC_REQUIRE(width == 16 || width == 32, MOC_ERR_ARG, "moc_plan_row_table: width %d (16 or 32)", width);
  MOC_REQUIRE(max_u >= 0 && max_u < ((int64_t)1 << 25), MOC_ERR_ARG, "moc_plan_row_table: max_u %lld",
              (long long)max_u);
  if (max_u == 0) return MOC_OK;
  hipLaunchKernelGGL(decode_row_table_kernel, dim3((unsigned)((max_u * width + 255) / 256)), dim3(256), 0, stream,
                     n_uniq, csr_off, csr_edge, max_u, width, row_tab);
  return check_launch("decode_row_table_kernel");
}

int moc_decode_row_table(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                         int32_t* row_tab, hipStream_t stream) {
  return moc_plan_row_table(n_uniq, csr_off, csr_edge, max_u, 16, row_tab, stream);
}

int moc_decode_partial(int dtype, const void* q, int64_t B, int H, const void* k_tiles, const void* v_tiles, int HK,
                       int Dh, int T, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                       const int32_t* csr_edge, int64_t max_u, const float* omega, int NS, float scale, void* o_part,
                       float* lse_part, const int32_t* row_tab, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && uniq && n_uniq && csr_off && csr_edge && omega && o_part && lse_part,
              MOC_ERR_ARG, "moc_decode_partial: null pointer");
  MOC_REQUIRE(Dh == 64 && T == 64, MOC_ERR_UNSUPPORTED, "moc_decode_partial: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0, MOC_ERR_ARG, "moc_decode_partial: bad heads");
  if (B == 0 || max_u == 0) return MOC_OK;
  // tiles [chapter][HK][64 keys][64 dims]; edge e = b * NS + slot serves query heads 0 .. H-1
  return sparse_fwd_launch(dtype, q, H, k_tiles, v_tiles, (int64_t)HK * 4096, 4096, 64, HK, uniq, n_uniq, csr_off,
                           csr_edge, max_u, NS, 0, HK, 0, H, scale, omega, o_part, lse_part, stream,
                           "moc_decode_partial", row_tab);
}

}  // extern "C"
