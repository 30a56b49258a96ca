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
// reads).  moc_sparse_combine (joint mode, rpe = H) merges the slots of a sequence.
#include "moc_common.h"

using namespace moc;

extern "C" {

int moc_decode_partial(int dtype, const void* q, int64_t B, int H, const void* k_tiles, const void* v_tiles, int HK,
                       int Dh, int T, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                       const int32_t* csr_edge, int64_t max_u, const float* omega, int NS, float scale, float* o_part,
                       float* lse_part, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && v_tiles && uniq && n_uniq && csr_off && csr_edge && omega && o_part && lse_part,
              MOC_ERR_ARG, "moc_decode_partial: null pointer");
  MOC_REQUIRE(Dh == 64 && T == 64, MOC_ERR_UNSUPPORTED, "moc_decode_partial: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0, MOC_ERR_ARG, "moc_decode_partial: bad heads");
  if (B == 0 || max_u == 0) return MOC_OK;
  // tiles [chapter][HK][64 keys][64 dims]; edge e = b * NS + slot serves query heads 0 .. H-1
  return sparse_fwd_launch(dtype, q, H, k_tiles, v_tiles, (int64_t)HK * 4096, 4096, 64, HK, uniq, n_uniq, csr_off,
                           csr_edge, max_u, NS, 0, HK, 0, H, scale, omega, o_part, lse_part, stream,
                           "moc_decode_partial");
}

}  // extern "C"
