// Shared device/host helpers for libmoc (MI355X / gfx950 only).
//
// Conventions used by every kernel in this library:
//  * Element types: T in {float, __bf16}.  All matrix products accumulate in
//    fp32 on the matrix cores (v_mfma_f32_16x16x32_bf16 for bf16 operands,
//    eight v_mfma_f32_16x16x4_f32 for fp32 operands).
//  * A "fragment" is 8 consecutive reduction-dimension (k) elements held by
//    one lane.  For the 16x16 MFMA tile, lane l holds row/column (l % 16) and
//    k-group g = l / 16 of the 32-wide k step.  The order of k inside one MFMA
//    reduction is free, so both operands only have to agree on it.
//  * Accumulator layout (16x16 fp32 tile, 4 values per lane):
//    lane l holds column n = l % 16 and rows m = 4 * (l / 16) + e, e = 0..3.
//  * Entry points never allocate and never synchronise the host; they return
//    a status code and keep a thread-local message for moc_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/moc.h"

namespace moc {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// ----------------------------------------------------------------- errors (host)
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define MOC_REQUIRE(cond, code, ...)                                   \
  do {                                                                 \
    if (!(cond)) return ::moc::set_error((code), __VA_ARGS__);         \
  } while (0)

#define MOC_HIP(call)                                                  \
  do {                                                                 \
    hipError_t _e = (call);                                            \
    if (_e != hipSuccess)                                              \
      return ::moc::set_error(MOC_ERR_LAUNCH, "%s: %s", #call,         \
                              hipGetErrorString(_e));                  \
  } while (0)

// Host check of a K / V block layout of the attention entry points: element (t, dh) of
// block (chapter slot u, kv head hk) at base + u * su + hk * sh + t * st + dh, each base
// readable for kv_span elements (bounded buffer loads).
inline int check_kv_layout(const char* who, int dtype, int64_t kv_span, int64_t su, int64_t sh, int64_t st) {
  const int64_t es = dtype == MOC_F32 ? 4 : 2;
  MOC_REQUIRE(kv_span > 0 && kv_span * es < ((int64_t)1 << 32), MOC_ERR_UNSUPPORTED,
              "%s: K / V buffers must be < 4 GiB (kv_span=%lld)", who, (long long)kv_span);
  MOC_REQUIRE(st >= 64 && sh >= 0 && su >= 0 && (st * es) % 16 == 0 && (sh * es) % 16 == 0 && (su * es) % 16 == 0,
              MOC_ERR_ARG, "%s: K / V strides (%lld, %lld, %lld) must be 16-byte multiples, row stride >= 64", who,
              (long long)su, (long long)sh, (long long)st);
  return MOC_OK;
}

// Router weights below this floor are taken as zero by the sequence-routed attention kernels,
// which fold omega into the exp2 argument through log2(omega) and 1 / omega: for a denormal
// omega those are -inf / inf (NaN once multiplied by a zero).  Below the floor the slot's keys
// k~ = omega k make every logit 0 to fp32 precision and its values and dQ terms are O(omega), so
// the zero-weight limit (the denominator gains exp2(-m) per key, nothing else) is exact in fp32.
constexpr float kTinyOmega = 0x1p-64f;

// ------------------------------------------------------------ element helpers
template <typename T> struct Frag;
template <> struct Frag<bf16> { typedef bf16x8 type; };
template <> struct Frag<float> { typedef f32x8 type; };

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }

// c += a * b over one 32-wide k step (see the header comment for layouts).
__device__ __forceinline__ void mma(f32x4& c, const bf16x8& a, const bf16x8& b) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& c, const f32x8& a, const f32x8& b) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
}

// 16-byte vector of raw bits.
struct alignas(16) V16 { uint32_t w[4]; };

__device__ __forceinline__ V16 ld16(const void* p) { return *reinterpret_cast<const V16*>(p); }
__device__ __forceinline__ void st16(void* p, const V16& v) { *reinterpret_cast<V16*>(p) = v; }

// Load 8 consecutive elements of type TI and return them as 8 elements of T.
template <typename T, typename TI> struct Load8;
template <typename T> struct Load8<T, T> {
  static __device__ __forceinline__ typename Frag<T>::type run(const T* p) {
    return *reinterpret_cast<const typename Frag<T>::type*>(p);
  }
};
template <> struct Load8<bf16, float> {
  static __device__ __forceinline__ bf16x8 run(const float* p) {
    f32x8 v = *reinterpret_cast<const f32x8*>(p);
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (bf16)v[j];
    return r;
  }
};

template <typename T> __device__ __forceinline__ typename Frag<T>::type zero_frag() {
  typename Frag<T>::type z;
#pragma unroll
  for (int j = 0; j < 8; ++j) z[j] = from_f<T>(0.f);
  return z;
}

// ------------------------------------------------------------- LDS tile views
// A TILE is a square-ish block of ROWS x COLS elements of T stored row-major
// with the 16-byte chunks of every row XOR-swizzled by (row & 7): a fragment
// read (16 lanes, 16 consecutive rows, same column chunk) then touches 8
// distinct chunk slots instead of one bank group.  Requires >= 8 chunks/row.
template <typename T, int COLS>
struct SwzTile {
  static constexpr int kRowBytes = COLS * (int)sizeof(T);
  static constexpr int kChunks = kRowBytes / 16;
  static_assert(kChunks >= 8 && (kChunks & (kChunks - 1)) == 0, "row must be >= 8 pow2 chunks");
  __device__ static __forceinline__ int off(int row, int col) {
    int byte = col * (int)sizeof(T);
    int chunk = byte >> 4;
    return row * kRowBytes + (((chunk ^ (row & 7)) & (kChunks - 1)) << 4) + (byte & 15);
  }
  // 8 consecutive elements starting at (row, col), col multiple of 8/4 for bf16/f32 chunk sizes.
  __device__ static __forceinline__ typename Frag<T>::type frag(const char* base, int row, int col) {
    typename Frag<T>::type r;
    if constexpr (sizeof(T) == 2) {
      r = *reinterpret_cast<const bf16x8*>(base + off(row, col));
    } else {
      f32x4 lo = *reinterpret_cast<const f32x4*>(base + off(row, col));
      f32x4 hi = *reinterpret_cast<const f32x4*>(base + off(row, col + 4));
      r = f32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    return r;
  }
  // Two groups of 4 consecutive elements: (row, c0..c0+3) and (row, c1..c1+3).
  __device__ static __forceinline__ typename Frag<T>::type frag44(const char* base, int row, int c0, int c1) {
    typename Frag<T>::type r;
    if constexpr (sizeof(T) == 2) {
      bf16x4 a = *reinterpret_cast<const bf16x4*>(base + off(row, c0));
      bf16x4 b = *reinterpret_cast<const bf16x4*>(base + off(row, c1));
      r = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    } else {
      f32x4 a = *reinterpret_cast<const f32x4*>(base + off(row, c0));
      f32x4 b = *reinterpret_cast<const f32x4*>(base + off(row, c1));
      r = f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    return r;
  }
};

// 8 consecutive elements (16 bytes of bf16 / 32 bytes of fp32) as floats
template <typename TB> struct ChunkLoadF;
template <> struct ChunkLoadF<bf16> {
  static __device__ __forceinline__ void run(const bf16* p, float* o) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int x = 0; x < 8; ++x) o[x] = (float)v[x];
  }
};
template <> struct ChunkLoadF<float> {
  static __device__ __forceinline__ void run(const float* p, float* o) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int x = 0; x < 4; ++x) { o[x] = a[x]; o[4 + x] = b[x]; }
  }
};

// XCD-aware tile order.  Workgroups of a launch are dealt round-robin to the 8 XCDs,
// each with its own L2.  With a 1-D grid padded to a multiple of 8 (xcd_grid), tile
// t = (w % 8) * (gridDim.x / 8) + w / 8 gives every XCD a contiguous range of tile ids,
// so tiles that share inputs (numbered consecutively by the kernel) meet in one L2.
// Returns -1 for the padding workgroups.
__device__ __forceinline__ int64_t xcd_tile(int64_t n_tiles) {
  const int64_t w = blockIdx.x, per = gridDim.x / 8;
  const int64_t t = (w % 8) * per + w / 8;
  return t < n_tiles ? t : -1;
}
inline unsigned xcd_grid(int64_t n_tiles) { return (unsigned)((n_tiles + 7) / 8 * 8); }

// MFMA key order of transposed tiles.  The P^T / dS^T fragments that feed the PV-type
// products (16x16x32) hold, in lane group g, keys 4g..4g+3 and 16+4g..16+4g+3 of each
// 32-key group.  Transposed tiles (K^T, V^T, Q^T, dO^T) store their key axis in that
// order -- key 4g + e at position 8g + e, key 16 + 4g + e at 8g + 4 + e -- so every such
// fragment is one contiguous 16-byte read (Tile::frag at column 32 c + 8 g).
__host__ __device__ constexpr int mfma_key_pos(int k) {
  return (k & ~31) | ((k & 31) < 16 ? 8 * ((k & 15) >> 2) + (k & 3) : 8 * ((k & 15) >> 2) + 4 + (k & 3));
}
__host__ __device__ constexpr int mfma_pos_key(int p) {
  return (p & ~31) | (((p & 4) ? 16 : 0) + 4 * ((p & 31) >> 3) + (p & 3));
}

// Transposing fragment read (ds_read_b64_tr_b16) from a row-major bf16 LDS tile with
// layout Tile::off(row, col): lane l receives column cb + l % 16 at rows rb + 4g + e
// (elements e = 0..3) and rb + 16 + 4g + e (elements 4 + e), g = l / 16 -- the k order
// of the MFMA key order above, so the result pairs with P / dS fragments held in
// accumulator layout.  Each 16-lane group reads 4 rows x 16 columns per instruction;
// lane q of the group supplies the address of row q / 4, columns 4 (q % 4) .. + 3.
template <typename Tile>
__device__ __forceinline__ bf16x8 tr_frag_mk(const char* base, int rb, int cb, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s* lds_v4s;
  const int q = lane & 15;
  const int row = rb + 4 * (lane >> 4) + (q >> 2), col = cb + 4 * (q & 3);
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + Tile::off(row, col)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + Tile::off(row + 16, col)));
  const v4s v[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8, v);
}

// The same MFMA-key-order fragment for either element type: bf16 through the transposing
// read above, fp32 (no transposing read for 32-bit elements) element by element.
template <typename Tile, typename T>
__device__ __forceinline__ typename Frag<T>::type mk_frag(const char* base, int rb, int cb, int lane) {
  if constexpr (sizeof(T) == 2) {
    return tr_frag_mk<Tile>(base, rb, cb, lane);
  } else {
    f32x8 r;
    const int row = rb + 4 * (lane >> 4), col = cb + (lane & 15);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[e] = *reinterpret_cast<const float*>(base + Tile::off(row + e, col));
      r[4 + e] = *reinterpret_cast<const float*>(base + Tile::off(row + 16 + e, col));
    }
    return r;
  }
}

// Orders LDS accesses of one wave: everything before is visible to every lane of the
// wave after (LDS executes one wave's instructions in order; this keeps the compiler
// from moving accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left open), gfx9 encoding
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// -------------------------------------------------------------- buffer loads
// Raw buffer loads: SGPR resource + per-thread VGPR offset + uniform SGPR offset.
// The per-thread offset register is fixed for a kernel's lifetime, so in-flight
// prefetches never pin address registers that later code wants to reuse, and
// reads past `bytes` return zero.
struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Buf(const void* p, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000)) {}
  __device__ __forceinline__ V16 load16(uint32_t voff, uint32_t soff) const {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return __builtin_bit_cast(V16, v);
  }
};

// ------------------------------------------------------ 64x64 tile movement
// One contiguous 64 x 64 tile of T (e.g. a chapter-head K or V block) moved
// global -> registers -> LDS by NT threads; each thread owns NCHUNK 16-byte
// chunks.  store() keeps row = first index, store_t() writes the transpose.
template <typename T, int NT>
struct TileIO {
  static constexpr int EPC = 16 / (int)sizeof(T);
  static constexpr int CPR = 64 / EPC;             // chunks per row
  static constexpr int NCHUNK = (64 * CPR) / NT;   // per thread
  using Tile = SwzTile<T, 64>;
  V16 r[NCHUNK];
  __device__ __forceinline__ void load(const T* src, int tid) {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) r[i] = ld16(src + (size_t)(tid + NT * i) * EPC);
  }
  // tile at byte offset `tile_off` of buffer `b`
  __device__ __forceinline__ void load(const Buf& b, uint32_t tile_off, int tid) {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) r[i] = b.load16((uint32_t)(tid + NT * i) * 16u, tile_off);
  }
  // 64 rows of 64 elements, row r at byte offset blk_off + r * row_bytes of buffer `b`
  __device__ __forceinline__ void load_rows(const Buf& b, uint32_t blk_off, uint32_t row_bytes, int tid) {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const uint32_t q = (uint32_t)(tid + NT * i);
      r[i] = b.load16((q / CPR) * row_bytes + (q % CPR) * 16u, blk_off);
    }
  }
  __device__ __forceinline__ void store(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int q = tid + NT * i;
      st16(dst + Tile::off(q / CPR, (q % CPR) * EPC), r[i]);
    }
  }
  __device__ __forceinline__ void store_t(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int q = tid + NT * i;
      const int row = q / CPR, c0 = (q % CPR) * EPC;
      const T* v = reinterpret_cast<const T*>(&r[i]);
#pragma unroll
      for (int x = 0; x < EPC; ++x) *reinterpret_cast<T*>(dst + Tile::off(c0 + x, row)) = v[x];
    }
  }
};

// ------------------------------------------------------------ wave reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Reduce over the 4 lanes {l, l^16, l^32, l^48} that share a 16x16 column.
// max without the operand canonicalisation fmaxf needs in IEEE mode (NaN-propagating;
// three-input forms fuse into v_maximum3_f32)
__device__ __forceinline__ float fmax_fast(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float quad_max(float v) {
  v = fmax_fast(v, __shfl_xor(v, 16, 64));
  v = fmax_fast(v, __shfl_xor(v, 32, 64));
  return v;
}
__device__ __forceinline__ float quad_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

inline int dtype_size(int dt) { return dt == MOC_F32 ? 4 : (dt == MOC_BF16 ? 2 : 0); }

// Chapter-centric partial attention of the token-routed path (sparse_xattn.hip), shared
// with the decode step: per (distinct chapter, kv head) unit, every row of every edge of
// the chapter gets o_part (normalised, times omega[e]) and lse_part (log2 domain) over
// the chapter's 64 keys, with logits scaled by omega[e] * scale (omega == nullptr: 1;
// omega >= 0).  Arguments as moc_sparse_fwd; `who` names the caller in errors.  row_tab
// (optional, i32 [max_u][16]): the first 16 edges of each distinct chapter (-1 padded,
// moc_decode_row_table), read instead of csr_edge for a unit's first 16 rows.
int sparse_fwd_launch(int dtype, const void* q, int HQ, const void* k, const void* v, int64_t cs, int64_t hs,
                      int64_t rs, int HK, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                      const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk, int hq_off, int rpe,
                      float scale, const float* omega, void* o_part, float* lse_part, hipStream_t stream,
                      const char* who, const int32_t* row_tab = nullptr);

// out[i] = inv * sum_j part[j * n + i] for i < n, j < nsplit, summed in a fixed order
// (router.hip's split-row reduction); returns a MOC_ status.
int launch_split_reduce(const float* part, int nsplit, int64_t n, float inv, float* out, hipStream_t stream);

// moc_chapter_wgrad with its grid held to `budget` workgroups (1..256), leaving the rest of the
// chip to work on other streams (the layer's router backward beside the K/V weight gradient)
int chapter_wgrad_budget(const void* dkv_edge, int64_t lda, const void* red, const void* x, int64_t ldx, int gather,
                         const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                         const int32_t* csr_edge, int N, int K, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                         int budget, hipStream_t stream);

// The chapters of a plan with several edges (the shared chapter, collisions), listed once per
// plan so that the per-chapter sums of their dK|dV rows need no scan of the inverted index:
// list[0] = count, entry i at list + 4 + kMultiEntry i: (u, cnt, p0, 0, first 8 edge ids (-1
// padded)).  dkv_multi_list: one workgroup (entries in any order; every sum below is fixed
// order).  dkv_multi_reduce_list: red[u] = sum of the listed chapters' edge rows, as
// moc_dkv_multi_reduce computes them (edges past the first 8 read from csr_edge + p0).
constexpr int kMultiEntry = 12;
inline size_t dkv_multi_list_bytes(int64_t max_u) { return (size_t)(4 + kMultiEntry * max_u) * 4; }
int dkv_multi_list(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                   int32_t* list, hipStream_t stream);
int dkv_multi_reduce_list(const void* dkv_edge, int64_t ld, const int32_t* list, int64_t max_u,
                          const int32_t* csr_edge, void* red, hipStream_t stream);

}  // namespace moc
