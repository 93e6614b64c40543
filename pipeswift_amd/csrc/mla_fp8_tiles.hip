// FP8 MLA latent entries with one float32 scale per 128-element tile: the
// append that writes them and the gather that reads them back.
//
// The reference keeps the MLA latent cache in bf16 and rejects FP8 for MLA
// models because their reader expects this other scheme, "per-128-element tiles
// with scales appended to the cache entry" (pipeswift/utils/arguments.py:459-467):
// the entry FlashMLA reads for an FP8 latent cache.  One entry holds
//   [0, nope_len)                     E4M3FN bytes of kv_c, tile j scaled by s_j
//   [nope_len, nope_len + 4*tiles)    s_j as float32, tiles = nope_len / 128
//   [rope_off, rope_off + 2*rope_len) k_pe as bf16 bit copies
// with rope_off = nope_len + 4*tiles (656 bytes for DeepSeek-V3: 512 + 16 + 128).
//
// Mapping on CDNA4: one wave64 per token.  A pass covers 4 tiles: lane l holds
// 8 elements of tile l/16, so a tile's amax is a max over one 16-lane DPP row
// (4 row-local DPP steps, no LDS), and every row stores its 128 bytes of E4M3
// plus one scale.  The rope part is copied by the first lanes in 16-byte
// vectors.  Loads and stores are nontemporal: each byte is touched once.

#include "psk_common.h"

using namespace psk_detail;

namespace {

constexpr int kTileElems = 128;
constexpr int kTilesPerPass = 4;  // 64 lanes x 8 elements
constexpr int kPassElems = kTileElems * kTilesPerPass;
constexpr int kWaves = 4;         // tokens per workgroup
constexpr int kMaxTiles = 64;     // nope_len <= 8192
constexpr float kMinScale = 0x1p-126f;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppRowMirror = 0x140;   // lane i <-> 15 - i within each 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xF, 0xF, false));
}

// Max over the 16 lanes of a DPP row; every lane of the row gets it.  On the
// bits of non-negative floats (no NaN), whose integer order is their order.
__device__ __forceinline__ uint32_t row16_max_bits(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  return max(v, dpp_u32<kDppRowMirror>(v));
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// max |x| over 8 bf16 elements as float32 bits, NaN ignored (it never wins
// the max).  The magnitudes are 15-bit integers whose order is the order of
// |x| up to +inf (0x7F80); NaNs sort above it.  Packed 16-bit maxima take two
// elements per instruction, and only a lane whose maximum is a NaN pattern
// takes the element-wise pass that skips NaNs.
__device__ __forceinline__ uint32_t amax8_bits(u32x4 x) {
  u16x2 m2 = {0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, x[i] & 0x7FFF7FFFu));
  uint32_t m = m2[0] > m2[1] ? m2[0] : m2[1];
  if (__builtin_expect(m > 0x7F80u, 0)) {
    m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = (x[i >> 1] >> (16 * (i & 1))) & 0x7FFFu;
      m = (v <= 0x7F80u && v > m) ? v : m;
    }
  }
  return m << 16;
}

// s = max(amax / 448, 2^-126) with the correctly rounded quotient.  From 2^-90
// up, Markstein's correction of amax * RN(1/448) is exact (no underflow in the
// residual); below, the IEEE division runs (never, for real activations).
__device__ __forceinline__ float tile_scale(float amax) {
  QScale k;
  k.s = 448.0f;
  k.r = 1.0f / 448.0f;
  k.fast = true;
  k.neg = 0u;
  const float q = amax >= 0x1p-90f ? div_fast(amax, k) : amax / 448.0f;
  return __builtin_fmaxf(q, kMinScale);
}

struct TileAppendArgs {
  const char* kv_c;
  const char* k_pe;
  char* cache;
  const int64_t* slots;
  int64_t num_tokens;
  int64_t num_slots;
  int64_t block_size;
  int64_t kv_c_stride;  // bytes
  int64_t k_pe_stride;  // bytes
  int64_t blk_stride;   // bytes
  int64_t page_stride;  // bytes
  int32_t bs_shift;     // log2(block_size), or -1
  int32_t tiles;
  int32_t rope_vecs;    // rope vectors of RV bytes
  int32_t rope_off;     // bytes from the entry start
};

// RV: bytes per rope vector; NV: bytes per E4M3 store (8, or 4 when entries
// are only 4-byte aligned).  WHOLE: the DeepSeek-V3 entry (4 tiles, 16 scale
// bytes, 128 rope bytes: 656 bytes on 16-byte boundaries), written by one
// store instruction of 16 bytes per lane over the whole entry.  An entry then
// leaves the L1 as one write request per 64-byte line it touches (11), so only
// the two lines it shares with its neighbours are partial; written as three
// parts (E4M3, scales, rope), the lines where the parts meet are split into
// separate partial requests too (12.5 per entry).
template <int RV, int NV, bool WHOLE = false>
__global__ void __launch_bounds__(kWaves * 64) tile_fp8_append_kernel(TileAppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t_wave = int64_t(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  // No early exit before the loads: a wave past the last token reads the last
  // token's row (num_tokens >= 1) and leaves at the slot check, so every
  // kernel argument is fetched in one round.
  const bool live = t_wave < a.num_tokens;
  const int64_t t = live ? t_wave : a.num_tokens - 1;
  const int64_t slot = a.slots[t];
  // The first pass of kv_c and the first rope vectors depend on t only: load
  // them before the slot arrives, so the two loads overlap instead of queueing.
  const char* src = a.kv_c + t * a.kv_c_stride;
  const char* pe = a.k_pe + t * a.k_pe_stride;
  u32x4 x0 = {0u, 0u, 0u, 0u};
  if ((lane >> 4) < a.tiles) x0 = vload_nt<16>(src + lane * 16);
  typename VecT<RV>::T r0 = 0;
  if (lane < a.rope_vecs) r0 = vload_nt<RV>(pe + lane * RV);
  if (!live || slot < 0 || slot >= a.num_slots) return;  // padding / foreign token
  int64_t blk, off;
  if (a.bs_shift >= 0) {
    blk = slot >> a.bs_shift;
    off = slot & (a.block_size - 1);
  } else {
    blk = slot / a.block_size;
    off = slot - blk * a.block_size;
  }
  char* entry = a.cache + blk * a.blk_stride + off * a.page_stride;
  const int nope_bytes = a.tiles * kTileElems;

  if constexpr (!WHOLE) {
    if (lane < a.rope_vecs) vstore_nt<RV>(entry + a.rope_off + lane * RV, r0);
  }
  for (int i = lane + 64; i < a.rope_vecs; i += 64) vstore_nt<RV>(entry + a.rope_off + i * RV, vload_nt<RV>(pe + i * RV));
  for (int p = 0; p * kTilesPerPass < a.tiles; ++p) {
    const int tile = p * kTilesPerPass + (lane >> 4);
    const bool active = tile < a.tiles;  // uniform over each 16-lane row
    const int e = p * kPassElems + lane * 8;
    u32x4 x = x0;
    if (p > 0) {
      x = u32x4{0u, 0u, 0u, 0u};
      if (active) x = vload_nt<16>(src + int64_t(e) * 2);
    }
    // every lane takes part in the row max (inactive rows reduce zeros)
    const float s = tile_scale(__uint_as_float(row16_max_bits(amax8_bits(x))));
    if (active) {
      // NaN inputs store 0x7F with their sign (kNanTorch), as the tile's own
      // rule has it
      const QScale qs = make_qscale(s);
      u32x2 q = QuantConv<PSK_DTYPE_BF16, 8, kNanTorch>::apply(x, qs);
      if (__builtin_expect(__builtin_isinf(s), 0)) {
        // A tile holding an infinity has s = inf, and +-inf / inf is a NaN
        // whose sign the division does not define: store 0x7F with the sign
        // of the input, as a NaN input stores.  Finite inputs give +-0.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t h = (x[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          if ((h & 0x7FFFu) == 0x7F80u) {
            const int sh = 8 * (i & 3);
            q[i >> 2] = (q[i >> 2] & ~(0xFFu << sh)) | ((((h >> 8) & 0x80u) | 0x7Fu) << sh);
          }
        }
      }
      if constexpr (WHOLE) {
        // one pass, every lane active: lane j < 32 takes the E4M3 bytes of
        // lanes 2j and 2j + 1, lane 32 the four scales (rows 0..3), lanes
        // 33..40 the rope vectors of lanes 0..7
        const uint32_t n0 = uint32_t(__shfl(int(q[0]), 2 * lane)), n1 = uint32_t(__shfl(int(q[1]), 2 * lane));
        const uint32_t n2 = uint32_t(__shfl(int(q[0]), 2 * lane + 1)), n3 = uint32_t(__shfl(int(q[1]), 2 * lane + 1));
        const int rl = lane - 33;
        const u32x4 rope = __builtin_bit_cast(u32x4, r0);
        const uint32_t r0w = uint32_t(__shfl(int(rope[0]), rl)), r1w = uint32_t(__shfl(int(rope[1]), rl));
        const uint32_t r2w = uint32_t(__shfl(int(rope[2]), rl)), r3w = uint32_t(__shfl(int(rope[3]), rl));
        const uint32_t sb = __float_as_uint(s);
        const u32x4 sc = {uint32_t(__builtin_amdgcn_readlane(int(sb), 0)), uint32_t(__builtin_amdgcn_readlane(int(sb), 16)),
                          uint32_t(__builtin_amdgcn_readlane(int(sb), 32)), uint32_t(__builtin_amdgcn_readlane(int(sb), 48))};
        const u32x4 w = lane < 32 ? u32x4{n0, n1, n2, n3} : lane == 32 ? sc : u32x4{r0w, r1w, r2w, r3w};
        if (lane <= 40) vstore_nt<16>(entry + 16 * lane, w);
      } else {
        if constexpr (NV == 8) {
          vstore_nt<8>(entry + e, q);
        } else {
          vstore_nt<4>(entry + e, q[0]);
          vstore_nt<4>(entry + e + 4, q[1]);
        }
        if ((lane & 15) == 0) vstore_nt<4>(entry + nope_bytes + 4 * tile, __float_as_uint(s));
      }
    }
  }
}

struct TileGatherArgs {
  const char* cache;
  char* dst;
  const int32_t* block_table;
  const int32_t* cu;
  const int32_t* starts;
  int64_t batch;
  int64_t bt_stride;
  int64_t num_tokens;
  int64_t block_size;
  int64_t num_blocks;
  int64_t blk_stride;   // bytes
  int64_t page_stride;  // bytes
  int64_t dst_stride;   // bytes
  int32_t bs_shift;
  int32_t tiles;
  int32_t rope_vecs;    // rope vectors of RV bytes (bf16 in the cache)
  int32_t rope_off;
};

// bf16 bits -> the output element type
template <int OUT_DT, int RV>
__device__ __forceinline__ void store_rope(char* out, typename VecT<RV>::T v) {
  if constexpr (OUT_DT == PSK_DTYPE_BF16) {
    vstore_nt<RV>(out, v);
  } else {
    constexpr int E = RV / 2;
    uint16_t h[E];
    __builtin_memcpy(h, &v, RV);
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      u32x2 w = {uint32_t(h[i]) << 16, uint32_t(h[i + 1]) << 16};
      vstore_nt<8>(out + 4 * i, w);
    }
  }
}

template <int OUT_DT, int RV, int NV>
__global__ void __launch_bounds__(kWaves * 64) tile_fp8_gather_kernel(TileGatherArgs g) {
  constexpr int osz = Elt<OUT_DT>::kSize;
  const int lane = threadIdx.x & 63;
  const int64_t t = int64_t(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  if (t >= g.num_tokens) return;
  // sequence of the token: largest b in [0, batch] with cu[b] <= t
  int lo = 0, hi = int(g.batch);
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(g.cu[mid]) <= t) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  if (b >= g.batch || t < int64_t(g.cu[0])) return;  // beyond the last sequence: untouched
  const int64_t p = (g.starts ? int64_t(g.starts[b]) : 0) + t - int64_t(g.cu[b]);
  int64_t page, off;
  if (g.bs_shift >= 0) {
    page = p >> g.bs_shift;
    off = p & (g.block_size - 1);
  } else {
    page = p / g.block_size;
    off = p - page * g.block_size;
  }
  int64_t blk = -1;
  if (p >= 0 && page < g.bt_stride) blk = g.block_table[int64_t(b) * g.bt_stride + page];
  const bool rd = blk >= 0 && blk < g.num_blocks;
  const char* entry = g.cache + (rd ? blk * g.blk_stride + off * g.page_stride : 0);
  char* out = g.dst + t * g.dst_stride;
  const int nope = g.tiles * kTileElems;

  for (int pass = 0; pass * kTilesPerPass < g.tiles; ++pass) {
    const int tile = pass * kTilesPerPass + (lane >> 4);
    if (tile >= g.tiles) continue;
    const int e = pass * kPassElems + lane * 8;
    u32x2 q = {0u, 0u};
    QScale qs;
    qs.s = 0.0f;
    qs.r = 0.0f;
    qs.fast = false;
    qs.neg = 0u;
    if (rd) {
      if constexpr (NV == 8) {
        q = vload_nt<8>(entry + e);
      } else {
        q[0] = vload_nt<4>(entry + e);
        q[1] = vload_nt<4>(entry + e + 4);
      }
      qs.s = __uint_as_float(vload<4>(entry + nope + 4 * tile));
    }
    if constexpr (OUT_DT == PSK_DTYPE_BF16) {
      vstore_nt<16>(out + int64_t(e) * osz, DequantConv<OUT_DT, 8>::apply(q, qs));
    } else {
      vstore_nt<16>(out + int64_t(e) * osz, DequantConv<OUT_DT, 4>::apply(q[0], qs));
      vstore_nt<16>(out + int64_t(e) * osz + 16, DequantConv<OUT_DT, 4>::apply(q[1], qs));
    }
  }
  for (int i = lane; i < g.rope_vecs; i += 64) {
    typename VecT<RV>::T r = 0;
    if (rd) r = vload_nt<RV>(entry + g.rope_off + i * RV);
    store_rope<OUT_DT, RV>(out + int64_t(nope + i * (RV / 2)) * osz, r);
  }
}

// Shared argument checks; returns PSK_OK and the rope vector width.
int check_tiles(int64_t nope_len, int64_t rope_len, int* tiles, int* rope_off) {
  if (nope_len <= 0 || nope_len % kTileElems || nope_len / kTileElems > kMaxTiles)
    return fail(PSK_E_ARG, "nope_len %lld must be a positive multiple of %d, at most %d", (long long)nope_len,
                kTileElems, kTileElems * kMaxTiles);
  if (rope_len < 0 || rope_len % 2 || 2 * rope_len > 64 * 16)
    return fail(PSK_E_ARG, "rope_len %lld must be even and at most 512", (long long)rope_len);
  *tiles = int(nope_len / kTileElems);
  *rope_off = int(nope_len + 4 * *tiles);
  return PSK_OK;
}

}  // namespace

extern "C" {

int64_t psk_mla_fp8_tile_entry_bytes(int64_t nope_len, int64_t rope_len) {
  g_err[0] = 0;
  int tiles, rope_off;
  const int st = check_tiles(nope_len, rope_len, &tiles, &rope_off);
  if (st != PSK_OK) return st;
  return rope_off + 2 * rope_len;
}

int psk_concat_and_cache_mla_fp8_tiles(const void* kv_c, const void* k_pe, void* kv_cache,
                                       const int64_t* slot_mapping, int64_t num_tokens, int64_t nope_len,
                                       int64_t rope_len, int64_t kv_c_stride, int64_t k_pe_stride,
                                       int64_t block_size, int64_t num_blocks, int64_t cache_block_stride,
                                       int64_t cache_page_stride, int in_dtype, void* stream) {
  begin_device_call();
  int tiles = 0, rope_off = 0;
  int st = check_tiles(nope_len, rope_len, &tiles, &rope_off);
  if (st != PSK_OK) return st;
  if (num_tokens < 0 || block_size <= 0 || num_blocks < 0 || kv_c_stride < 0 || k_pe_stride < 0 ||
      cache_block_stride < 0 || cache_page_stride < 0)
    return fail(PSK_E_ARG, "bad sizes: num_tokens=%lld block_size=%lld num_blocks=%lld", (long long)num_tokens,
                (long long)block_size, (long long)num_blocks);
  if (in_dtype != PSK_DTYPE_BF16) return fail(PSK_E_DTYPE, "tile-scaled FP8 MLA entries take bf16 input (got %d)", in_dtype);
  const int64_t entry = rope_off + 2 * rope_len;
  if (cache_page_stride < entry && block_size > 1)
    return fail(PSK_E_ARG, "cache page stride %lld is shorter than the %lld-byte entry", (long long)cache_page_stride,
                (long long)entry);
  if (num_tokens == 0 || num_blocks == 0) return PSK_OK;
  if (!kv_c || !kv_cache || !slot_mapping || (rope_len > 0 && !k_pe)) return fail(PSK_E_ARG, "NULL tensor pointer");
  const uint64_t in_v[2] = {uint64_t(uintptr_t(kv_c)), uint64_t(kv_c_stride * 2)};
  if (common_align(in_v, 2, 16) < 16) return fail(PSK_E_ARG, "kv_c rows must start on 16-byte boundaries");
  const uint64_t ent_v[3] = {uint64_t(uintptr_t(kv_cache)), uint64_t(cache_block_stride), uint64_t(cache_page_stride)};
  const int nv = common_align(ent_v, 3, 8);
  if (nv < 4) return fail(PSK_E_ARG, "cache entries must start on 4-byte boundaries");
  const uint64_t rope_v[6] = {uint64_t(uintptr_t(k_pe)), uint64_t(k_pe_stride * 2), ent_v[0], ent_v[1], ent_v[2],
                              uint64_t(rope_off) | uint64_t(2 * rope_len)};
  const int rv = rope_len > 0 ? common_align(rope_v, 6, 16) : 16;

  TileAppendArgs a;
  a.kv_c = static_cast<const char*>(kv_c);
  a.k_pe = static_cast<const char*>(k_pe);
  a.cache = static_cast<char*>(kv_cache);
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.num_slots = num_blocks * block_size;
  a.block_size = block_size;
  a.kv_c_stride = kv_c_stride * 2;
  a.k_pe_stride = k_pe_stride * 2;
  a.blk_stride = cache_block_stride;
  a.page_stride = cache_page_stride;
  a.bs_shift = log2_exact(block_size);
  a.tiles = tiles;
  a.rope_vecs = int(2 * rope_len / rv);
  a.rope_off = rope_off;
  const dim3 grid(unsigned(ceil_div(num_tokens, kWaves))), block(kWaves * 64);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define PSK_TILE_APPEND(RV)                                                       \
  if (nv == 8) hipLaunchKernelGGL((tile_fp8_append_kernel<RV, 8>), grid, block, 0, s, a); \
  else hipLaunchKernelGGL((tile_fp8_append_kernel<RV, 4>), grid, block, 0, s, a)
  // the DeepSeek-V3 entry on 16-byte boundaries, prefill-sized batches: one
  // store over the entry (config 4 prefill 4.33 -> 4.20 us, HBM bytes 1.059x
  // -> 1.032x the algorithmic).  A decode-sized batch is latency bound, and the
  // lane exchange that assembles the entry lengthens its critical path (128
  // tokens: 2.68 -> 2.74 us), so it keeps the three-part stores.
  const bool whole = num_tokens >= 1024 && tiles == kTilesPerPass && rope_off == kPassElems + 4 * kTilesPerPass &&
                     2 * rope_len == 128 && rv == 16 && common_align(ent_v, 3, 16) == 16;
  if (whole) {
    hipLaunchKernelGGL((tile_fp8_append_kernel<16, 8, true>), grid, block, 0, s, a);
    return check_launch("tile_fp8_append_kernel launch");
  }
  switch (rv) {
    case 16: PSK_TILE_APPEND(16); break;
    case 8: PSK_TILE_APPEND(8); break;
    case 4: PSK_TILE_APPEND(4); break;
    default: PSK_TILE_APPEND(2); break;
  }
#undef PSK_TILE_APPEND
  return check_launch("tile_fp8_append_kernel launch");
}

int psk_gather_mla_fp8_tiles(const void* kv_cache, void* dst, const int32_t* block_table,
                             const int32_t* cu_seq_lens, const int32_t* seq_starts, int64_t batch_size,
                             int64_t block_table_stride, int64_t num_tokens, int64_t nope_len, int64_t rope_len,
                             int64_t block_size, int64_t num_blocks, int64_t cache_block_stride,
                             int64_t cache_page_stride, int64_t dst_row_stride, int out_dtype, void* stream) {
  begin_device_call();
  int tiles = 0, rope_off = 0;
  int st = check_tiles(nope_len, rope_len, &tiles, &rope_off);
  if (st != PSK_OK) return st;
  if (batch_size < 0 || num_tokens < 0 || block_size <= 0 || num_blocks < 0 || block_table_stride < 0 ||
      cache_block_stride < 0 || cache_page_stride < 0 || dst_row_stride < 0)
    return fail(PSK_E_ARG, "bad sizes: batch=%lld num_tokens=%lld block_size=%lld", (long long)batch_size,
                (long long)num_tokens, (long long)block_size);
  if (out_dtype != PSK_DTYPE_BF16 && out_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "tile-scaled FP8 MLA gather writes bf16 or f32 (got %d)", out_dtype);
  const int osz = out_dtype == PSK_DTYPE_F32 ? 4 : 2;
  if (dst_row_stride < (nope_len + rope_len) * osz && num_tokens > 1)
    return fail(PSK_E_ARG, "dst row stride %lld bytes is shorter than a row", (long long)dst_row_stride);
  if (num_tokens == 0 || batch_size == 0) return PSK_OK;
  if (!kv_cache || !dst || !block_table || !cu_seq_lens) return fail(PSK_E_ARG, "NULL tensor pointer");
  const uint64_t ent_v[3] = {uint64_t(uintptr_t(kv_cache)), uint64_t(cache_block_stride), uint64_t(cache_page_stride)};
  const int nv = common_align(ent_v, 3, 8);
  if (nv < 4) return fail(PSK_E_ARG, "cache entries must start on 4-byte boundaries");
  const uint64_t dst_v[2] = {uint64_t(uintptr_t(dst)), uint64_t(dst_row_stride)};
  if (common_align(dst_v, 2, 16) < 16) return fail(PSK_E_ARG, "dst rows must start on 16-byte boundaries");
  // rope vectors of RV cache bytes; entries are 4-byte aligned and rope_off and
  // 2*rope_len are multiples of 4, so RV >= 4
  const uint64_t rope_v[4] = {ent_v[0], ent_v[1], ent_v[2], uint64_t(rope_off) | uint64_t(2 * rope_len)};
  const int rv = common_align(rope_v, 4, 16);

  TileGatherArgs g;
  g.cache = static_cast<const char*>(kv_cache);
  g.dst = static_cast<char*>(dst);
  g.block_table = block_table;
  g.cu = cu_seq_lens;
  g.starts = seq_starts;
  g.batch = batch_size;
  g.bt_stride = block_table_stride;
  g.num_tokens = num_tokens;
  g.block_size = block_size;
  g.num_blocks = num_blocks;
  g.blk_stride = cache_block_stride;
  g.page_stride = cache_page_stride;
  g.dst_stride = dst_row_stride;
  g.bs_shift = log2_exact(block_size);
  g.tiles = tiles;
  g.rope_vecs = rope_len > 0 ? int(2 * rope_len / rv) : 0;
  g.rope_off = rope_off;
  const dim3 grid(unsigned(ceil_div(num_tokens, kWaves))), block(kWaves * 64);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define PSK_TILE_GATHER(OUT, RV)                                                        \
  if (nv == 8) hipLaunchKernelGGL((tile_fp8_gather_kernel<OUT, RV, 8>), grid, block, 0, s, g); \
  else hipLaunchKernelGGL((tile_fp8_gather_kernel<OUT, RV, 4>), grid, block, 0, s, g)
  if (out_dtype == PSK_DTYPE_BF16) {
    switch (rv) {
      case 16: PSK_TILE_GATHER(PSK_DTYPE_BF16, 16); break;
      case 8: PSK_TILE_GATHER(PSK_DTYPE_BF16, 8); break;
      default: PSK_TILE_GATHER(PSK_DTYPE_BF16, 4); break;
    }
  } else {
    switch (rv) {
      case 16: PSK_TILE_GATHER(PSK_DTYPE_F32, 16); break;
      case 8: PSK_TILE_GATHER(PSK_DTYPE_F32, 8); break;
      default: PSK_TILE_GATHER(PSK_DTYPE_F32, 4); break;
    }
  }
#undef PSK_TILE_GATHER
  return check_launch("tile_fp8_gather_kernel launch");
}

}  // extern "C"
