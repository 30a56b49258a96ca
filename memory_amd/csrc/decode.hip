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
// decode_partial_kernel: one wave per (distinct chapter u, kv head hk).  Lane j
// holds key row j of the K tile and lane d value column d (row d of the V^T tile,
// whose key axis is in MFMA key order).
// For every edge (b, slot) of u and every query head hq of hk:
//   s_j = omega * scale * q . k_j  ->  lse (log2), o_d = omega * sum_j p_j v_jd / sum_j p_j
// written as partials; moc_sparse_combine (joint mode) merges the slots of a sequence.
#include "moc_common.h"

namespace moc {

constexpr int kDecWaves = 4;

template <typename T>
__global__ __launch_bounds__(64 * kDecWaves) void decode_partial_kernel(
    const T* __restrict__ q, int H, const T* __restrict__ ktiles, const T* __restrict__ vttiles, int HK,
    const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_uniq, const int32_t* __restrict__ csr_off,
    const int32_t* __restrict__ csr_edge, const float* __restrict__ omega, int NS, float scale_log2,
    float* __restrict__ o_part, float* __restrict__ lse_part) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t pair = (int64_t)blockIdx.x * kDecWaves + wave;
  const int nu = n_uniq[0];
  if (pair >= (int64_t)nu * HK) return;
  const int u = (int)(pair / HK), hk = (int)(pair % HK);
  const int gid = uniq[u];
  const size_t tile = ((size_t)gid * HK + hk) * 4096;
  // key row `lane` and value column `lane` (64 elements each)
  constexpr int EPC = 16 / (int)sizeof(T);
  float kr[64], vc[64];
  {
    const T* kp = ktiles + tile + (size_t)lane * 64;
    const T* vp = vttiles + tile + (size_t)lane * 64;
#pragma unroll
    for (int c = 0; c < 64 / EPC; ++c) {
      V16 a = ld16(kp + c * EPC);
      V16 b = ld16(vp + c * EPC);
      const T* ta = reinterpret_cast<const T*>(&a);
      const T* tb = reinterpret_cast<const T*>(&b);
#pragma unroll
      for (int x = 0; x < EPC; ++x) {
        kr[c * EPC + x] = to_f(ta[x]);
        vc[c * EPC + x] = to_f(tb[x]);
      }
    }
  }

  const int G = H / HK;
  const int p0 = csr_off[u], p1 = csr_off[u + 1];
  for (int p = p0; p < p1; ++p) {
    const int e = csr_edge[p];
    const int b = e / NS;
    const float w = omega[e];
    const float c = w * scale_log2;
    for (int hq = hk * G; hq < hk * G + G; ++hq) {
      const T* qp = q + ((size_t)b * H + hq) * 64;
      float dot = 0.f;
#pragma unroll
      for (int cc = 0; cc < 64 / EPC; ++cc) {
        V16 a = ld16(qp + cc * EPC);
        const T* ta = reinterpret_cast<const T*>(&a);
#pragma unroll
        for (int x = 0; x < EPC; ++x) dot += to_f(ta[x]) * kr[cc * EPC + x];
      }
      const float s = dot * c;
      const float m = wave_max(s);
      const float pj = __builtin_amdgcn_exp2f(s - m);
      const float l = wave_sum(pj);
      float o = 0.f;
#pragma unroll
      // vc[j] is V^T at position j of the MFMA key order, i.e. key mfma_pos_key(j)
      for (int j = 0; j < 64; ++j)
        o += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), mfma_pos_key(j))) * vc[j];
      const size_t row = (size_t)e * H + hq;
      o_part[row * 64 + lane] = o * (w / l);
      if (lane == 0) lse_part[row] = m + log2f(l);
    }
  }
}

}  // namespace moc

using namespace moc;

extern "C" {

int moc_decode_partial(int dtype, const void* q, int64_t B, int H, const void* k_tiles, const void* vt_tiles, int HK,
                       int Dh, int T, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                       const int32_t* csr_edge, int64_t max_u, const float* omega, int NS, float scale, float* o_part,
                       float* lse_part, hipStream_t stream) {
  MOC_REQUIRE(q && k_tiles && vt_tiles && uniq && n_uniq && csr_off && csr_edge && omega && o_part && lse_part,
              MOC_ERR_ARG, "moc_decode_partial: null pointer");
  MOC_REQUIRE(Dh == 64 && T == 64, MOC_ERR_UNSUPPORTED, "moc_decode_partial: needs head_dim 64 and T 64");
  MOC_REQUIRE(H > 0 && HK > 0 && H % HK == 0 && NS > 0, MOC_ERR_ARG, "moc_decode_partial: bad heads");
  if (B == 0 || max_u == 0) return MOC_OK;
  const int64_t pairs = max_u * HK;
  dim3 grid((unsigned)((pairs + kDecWaves - 1) / kDecWaves));
  const float sl2 = scale * 1.4426950408889634f;
  if (dtype == MOC_BF16)
    hipLaunchKernelGGL(decode_partial_kernel<bf16>, grid, dim3(64 * kDecWaves), 0, stream, (const bf16*)q, H,
                       (const bf16*)k_tiles, (const bf16*)vt_tiles, HK, uniq, n_uniq, csr_off, csr_edge, omega, NS, sl2,
                       o_part, lse_part);
  else if (dtype == MOC_F32)
    hipLaunchKernelGGL(decode_partial_kernel<float>, grid, dim3(64 * kDecWaves), 0, stream, (const float*)q, H,
                       (const float*)k_tiles, (const float*)vt_tiles, HK, uniq, n_uniq, csr_off, csr_edge, omega, NS,
                       sl2, o_part, lse_part);
  else
    return set_error(MOC_ERR_UNSUPPORTED, "moc_decode_partial: dtype %d", dtype);
  return check_launch("decode_partial_kernel");
}

}  // extern "C"
