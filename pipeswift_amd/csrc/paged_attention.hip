// Paged decode attention over the FP8 E4M3FN KV cache for MI355X (gfx950): the
// reader of what the append writes, with per-(sequence, kv head) descales.
//
// For sequence b, query head hq = h * G + g (G query heads per kv head h) and the
// first seq_lens[b] tokens j of the paged cache:
//   q~      = e4m3(q[b, hq] / qd)            (an FP8 query is taken as is)
//   s_j     = softmax_scale * qd * kd * (q~ . K[j, h])
//   out     = vd * sum_j softmax(s)_j V[j, h]
//   lse     = log(sum_j exp(s_j))
// with qd, kd, vd the descales of (b, h).  This is what the reference's decode
// reads through vLLM's FA3 fork (pipeswift/llms/layers/attention.py:148-187,
// FP8 query, descales per (sequence, kv head)); there the descales are fixed at
// 1.0 (pipeswift/utils/fp8_kv.py:94-103).
//
// Mapping (head_dim 128, one wave per 16-token tile of one kv head):
//   * Q K^T is one v_mfma_f32_16x16x32_bf16 chain of 4: the G query heads of
//     the group are rows (padded to 16), the tile's 16 tokens are columns.  Lane
//     l loads 32 contiguous bytes of token (l % 16)'s K row at d = 32 * (l / 16)
//     and the query operand uses the same d permutation.  Both operands are FP8
//     values converted exactly to bf16 (v_cvt_scalef32_pk_bf16_fp8 at scale 1),
//     so the products are exact and the sums are fp32.  The FP8 MFMA
//     (v_mfma_f32_16x16x32_fp8_fp8) is not used: on gfx950 it drops low-order
//     bits of small products against the largest one (measured: 256 + 31 * 2^-6
//     sums to 256.375), the accumulation loss the reference's FA3 fork has a
//     fix for on Hopper (pipeswift/utils/fp8_kv.py:6-13).
//   * softmax runs in the exp2 domain with a lazily raised running maximum
//     (raised only when a score exceeds it by 2^8), which keeps the rescaling of
//     the accumulators off the per-tile path; normalisation is exact.
//   * P V on the matrix cores, with S^T = K Q^T so that each lane holds one
//     head's scores of four tokens (the P operand), V^T read from LDS by
//     ds_read_b64_tr_b8, and P split into bf16 hi + lo (relative error 2^-17
//     per weight, fp32 sums); see "P V on the matrix cores" below.
//   * every tile goes through a per-wave ring of LDS slots filled by
//     global_load_lds, R tiles in flight per wave.  For power-of-two block
//     sizes >= 16 a tile lies in one page and is addressed wave-uniformly; for
//     any other block size each lane addresses its own rows (ring_attend's GEN
//     variant), so every block size takes the same kernels.
//   * schedules: the balanced one (equal runs of (sequence, tile) units per
//     workgroup across sequence boundaries, head-parallel from two sequences)
//     by default, or an explicit split count; the waves of a workgroup merge
//     through LDS into partial records (max, sum, accumulator per query head)
//     in the caller's workspace, and a second kernel merges a sequence's
//     records and writes the output.
//
// C ABI: include/pipeswift_kv.h.  Nothing here allocates or synchronizes.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <map>
#include <mutex>

#include "pipeswift_kv.h"
#include "psk_common.h"

using namespace psk_detail;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kHead = 128;    // head_dim of the MFMA tiling
constexpr int kTile = 16;     // tokens per tile (N of the 16x16x32 MFMA)
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kMinSplit = 256;
constexpr int kMaxSplits = 128;
// MFMA rows per (sequence, kv head): query tokens x query heads per kv head,
// padded to 1, 2, 4, 8 or 16 (16 with P V on the matrix cores)
constexpr int kMaxRows = 16;
constexpr float kNegBig = -1.0e30f;  // finite "no token yet" maximum
constexpr float kLazy = 8.0f;        // raise the running max past 2^8 headroom only
constexpr int kRing = 2;             // LDS tile slots per wave (ring kernel)
constexpr int kRingPages = 1024;     // page ids of a split in the ring kernel
// Sequences of the balanced schedule: every workgroup scans their lengths
// (twice) and keeps the prefix in the ring's LDS.
constexpr int kStreamMaxSeqs = 1024;
static_assert(kRingPages % (kWaves * 64) == 0, "page ids are staged a whole number per thread");

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

struct DecodeArgs {
  const char* q;
  int64_t q_tok_stride;   // bytes
  int64_t q_head_stride;  // bytes
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_blk, k_row, k_head;  // bytes
  int64_t v_blk, v_row, v_head;
  const int32_t* block_table;
  int64_t bt_stride;
  int64_t bt_width;
  const int32_t* seq_lens;
  int32_t num_blocks;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) or -1
  int32_t num_kv_heads;
  int32_t group;     // MFMA rows per (sequence, kv head): q_len query tokens x heads
  int32_t heads;     // query heads per kv head
  int32_t q_len;     // query token slots per sequence (the most query tokens any sequence has)
  const int32_t* cu_q;  // query tokens of sequence b: [cu_q[b], cu_q[b+1]); NULL: [b q_len, (b+1) q_len)
  int32_t causal;    // query token i of n of a sequence of length L sees keys [0, L - n + 1 + i)
  int32_t split;     // tokens per workgroup
  int32_t max_splits;
  float scale_log2;  // softmax_scale * log2(e)
  const float* qd;
  int64_t qd_b, qd_h;
  const float* kd;
  int64_t kd_b, kd_h;
  const float* vd;
  int64_t vd_b, vd_h;
  float* part;       // partial records of G * (kHead + 2) floats: [B][Hkv][max_splits] (splits) or
                     // [(B + stream_wgs) * Hkv] (balanced schedule)
  int32_t* prefix;   // balanced schedule: units before each sequence, [B + 1]
  int32_t stream_wgs;  // balanced schedule: workgroups per kv head; 0 with splits
  int32_t seq_units;   // balanced schedule: units that stand for the start of a sequence
  char* out;
  int64_t out_tok_stride;   // bytes
  int64_t out_head_stride;  // bytes
  float* lse;               // [Hq][lse_head_stride] (entry [hq][b]) or nullptr
  int64_t lse_head_stride;
};

// First query token of sequence b and how many it has (at most q_len).
__device__ __forceinline__ int64_t q_first(const DecodeArgs& a, int b) {
  return a.cu_q ? int64_t(a.cu_q[b]) : int64_t(b) * a.q_len;
}
__device__ __forceinline__ int q_count(const DecodeArgs& a, int b) {
  return a.cu_q ? max(0, min(a.q_len, a.cu_q[b + 1] - a.cu_q[b])) : a.q_len;
}

__device__ __forceinline__ float descale(const float* p, int64_t sb, int64_t sh, int b, int h) {
  return p ? p[b * sb + h * sh] : 1.0f;
}

// Eight E4M3FN bytes (w0 then w1, in byte order) -> eight bf16, exactly: every
// E4M3FN value is a bf16 value.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16(uint32_t w0, uint32_t w1) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The same to fp16, exactly: E4M3FN's 3-bit mantissas and exponents 2^-9 ..
// 2^8 (448 at most) all lie in fp16's range and precision.
__device__ __forceinline__ f16x8 e4m3x8_to_f16(uint32_t w0, uint32_t w1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppRowRor8 = 0x128;   // lane i <- lane (i + 8) % 16 within each row
constexpr int kDppRowMirror = 0x140;  // lane i <-> 15 - i within each row

// P V lane roles.  With replicated query rows (groups of at most 4 heads) lane
// l owns tokens (l % 8) and (l % 8) + 8 of a tile and V columns 16 * (l / 8) ..
// +16, so both of its tokens' scores sit in its own 16-lane row.  Otherwise
// tokens (l / 8) and (l / 8) + 8, columns 16 * (l % 8).
template <bool REPL>
__device__ __forceinline__ int token_slot(int lane) { return REPL ? (lane & 7) : (lane >> 3); }
template <bool REPL>
__device__ __forceinline__ int column_chunk(int lane) { return REPL ? (lane >> 3) : (lane & 7); }

__device__ __forceinline__ float bperm(int src_lane, float x) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(x)));
}

__device__ __forceinline__ int page_index(const DecodeArgs& a, int t) {
  return a.bs_shift >= 0 ? (t >> a.bs_shift) : (t / a.block_size);
}

// Page id of table entry pi, or -1 past the table's width or out of range.
__device__ __forceinline__ int32_t checked_page(const DecodeArgs& a, const int32_t* bt_row, int64_t pi) {
  if (pi >= a.bt_width) return -1;
  const int32_t p = bt_row[pi];
  return (p >= 0 && p < a.num_blocks) ? p : -1;
}

// Tile loads of one lane: K (32 bytes of one token) and V (16 bytes of two tokens).
struct TileLoads {
  u32x4 k0, k1, va, vb;
};

// 32 FP8 query bytes of this lane's MFMA row (query head h*G + lane%16, d from
// 32 * (lane / 16)); zero rows beyond the group.
template <int Q_DT>
__device__ __forceinline__ void load_query_as(const char* src, float qd, int d0, uint32_t qw[8]) {
  if constexpr (Q_DT == PSK_DTYPE_FP8_E4M3FN) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(src + d0);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(src + d0 + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qw[i] = lo[i];
      qw[4 + i] = hi[i];
    }
  } else {
    constexpr int kEsz = Elt<Q_DT>::kSize;
    constexpr int E = 16 / kEsz;  // elements per 16-byte load
    using QC = QuantConv<Q_DT, E, kNanTorch>;  // the query is quantized as fp8_kv.quantize does
    const QScale qs = make_qscale(qd);
    uint8_t bytes[32];
#pragma unroll
    for (int i = 0; i < 32 / E; ++i) {
      const typename QC::In x = *reinterpret_cast<const typename QC::In*>(src + (d0 + E * i) * kEsz);
      const typename QC::Out y = QC::apply(x, qs);
      __builtin_memcpy(bytes + E * i, &y, E);
    }
    __builtin_memcpy(qw, bytes, 32);
  }
}

// rows: MFMA row i holds query head i, or head i % 4 when REPL (groups of at
// most 4 heads repeated in each of the four row quarters)
template <bool REPL>
__device__ __forceinline__ void load_query(const DecodeArgs& a, int q_dtype, int b, int h, float qd, int lane,
                                           uint32_t qw[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) qw[i] = 0;
  const int row = REPL ? (lane & 3) : (lane & 15);
  if (row >= a.group) return;
  // row = i * heads + g: query token i of the sequence, head g of the group
  const int i = row / a.heads, g = row - i * a.heads;
  if (i >= q_count(a, b)) return;
  const char* src = a.q + (q_first(a, b) + i) * a.q_tok_stride + int64_t(h * a.heads + g) * a.q_head_stride;
  const int d0 = 32 * (lane >> 4);
  switch (q_dtype) {
    case PSK_DTYPE_FP8_E4M3FN: load_query_as<PSK_DTYPE_FP8_E4M3FN>(src, qd, d0, qw); break;
    case PSK_DTYPE_BF16: load_query_as<PSK_DTYPE_BF16>(src, qd, d0, qw); break;
    case PSK_DTYPE_F16: load_query_as<PSK_DTYPE_F16>(src, qd, d0, qw); break;
    default: load_query_as<PSK_DTYPE_F32>(src, qd, d0, qw); break;
  }
}

// Running softmax of one lane: per query head of the group the running
// maximum m (exp2 domain), its lazy threshold mth = m + kLazy, the sum l of
// exp2(s - m) and the weighted sum acc of the lane's 16 V columns.
template <int NG>
struct Softmax {
  float m[NG], mth[NG], l[NG], acc[NG][16];
};

// One 16-token tile of one wave.  The MFMA leaves S[g][t] in lane
// 16 * (g / 4) + t, register g % 4; the scores are scaled (and, in a PARTIAL
// tile, tokens at or past t_end masked to -inf) there, then each lane pulls the
// scores of its two tokens.  `consumed` runs as soon as the tile's K and V
// registers have been read (the caller starts the next loads there, so they fly
// during the softmax and P V).
template <int NG, bool PARTIAL, class Consumed>
__device__ __forceinline__ void attend_step(Softmax<NG>& st, TileLoads& c, const bf16x8 qop[4], float sl, int t0,
                                            int t_end, int lane, const Consumed& consumed) {
  constexpr bool REPL = NG <= 4;
  const int tv = token_slot<REPL>(lane);
  f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qop[0], e4m3x8_to_bf16(c.k0[0], c.k0[1]), sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qop[1], e4m3x8_to_bf16(c.k0[2], c.k0[3]), sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qop[2], e4m3x8_to_bf16(c.k1[0], c.k1[1]), sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qop[3], e4m3x8_to_bf16(c.k1[2], c.k1[3]), sc, 0, 0, 0);
  float fa[16], fb[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t wa = c.va[i], wb = c.vb[i];
    if constexpr (PARTIAL) {
      // rows past t_end may hold anything (a NaN would survive p = 0)
      wa = t0 + tv < t_end ? wa : 0u;
      wb = t0 + tv + 8 < t_end ? wb : 0u;
    }
    const f32x2 a0 = e4m3_unpack2(wa, false), a1 = e4m3_unpack2(wa, true);
    const f32x2 b0 = e4m3_unpack2(wb, false), b1 = e4m3_unpack2(wb, true);
    fa[4 * i] = a0.x;
    fa[4 * i + 1] = a0.y;
    fa[4 * i + 2] = a1.x;
    fa[4 * i + 3] = a1.y;
    fb[4 * i] = b0.x;
    fb[4 * i + 1] = b0.y;
    fb[4 * i + 2] = b1.x;
    fb[4 * i + 3] = b1.y;
  }
  consumed();

  float s4[4];
  const bool col_ok = !PARTIAL || t0 + (lane & 15) < t_end;
#pragma unroll
  for (int r = 0; r < 4; ++r) s4[r] = col_ok ? sc[r] * sl : -__builtin_inff();
  float sa[NG], sb[NG];
  bool raise = false;
  const bool low = (lane & 15) < 8;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if constexpr (REPL) {
      // this lane's column is one of its tokens; the other is 8 lanes away in the row
      const float own = s4[g], other = dpp<kDppRowRor8>(s4[g]);
      sa[g] = low ? own : other;
      sb[g] = low ? other : own;
    } else {
      sa[g] = bperm(16 * (g >> 2) + tv, s4[g & 3]);
      sb[g] = bperm(16 * (g >> 2) + tv + 8, s4[g & 3]);
    }
    raise |= __builtin_fmaxf(sa[g], sb[g]) > st.mth[g];
  }
  if (__any(raise)) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const float mn = __builtin_fmaxf(st.m[g], __builtin_fmaxf(sa[g], sb[g]));
      const float cr = __builtin_amdgcn_exp2f(st.m[g] - mn);
      st.l[g] *= cr;
#pragma unroll
      for (int k = 0; k < 16; ++k) st.acc[g][k] *= cr;
      st.m[g] = mn;
      st.mth[g] = mn + kLazy;
    }
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float pa = __builtin_amdgcn_exp2f(sa[g] - st.m[g]);
    const float pb = __builtin_amdgcn_exp2f(sb[g] - st.m[g]);
    st.l[g] += pa + pb;
#pragma unroll
    for (int k = 0; k < 16; ++k) st.acc[g][k] = __builtin_fmaf(pa, fa[k], __builtin_fmaf(pb, fb[k], st.acc[g][k]));
  }
}

// One merge step of the running softmax with the partner lane DPP pattern CTRL
// selects.
template <int NG, int CTRL>
__device__ __forceinline__ void merge_slots(Softmax<NG>& st) {
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float mo = dpp<CTRL>(st.m[g]);
    const float lo = dpp<CTRL>(st.l[g]);
    const float mn = __builtin_fmaxf(st.m[g], mo);
    const float ca = __builtin_amdgcn_exp2f(st.m[g] - mn), cb = __builtin_amdgcn_exp2f(mo - mn);
    st.l[g] = st.l[g] * ca + lo * cb;
#pragma unroll
    for (int k = 0; k < 16; ++k) st.acc[g][k] = st.acc[g][k] * ca + dpp<CTRL>(st.acc[g][k]) * cb;
    st.m[g] = mn;
  }
}

// Merge the wave's eight token slots, then the workgroup's waves through LDS,
// and write partial record `rec_idx`: per query head the maximum, the sum and
// the 128 weighted V columns.
template <int NG>
__device__ __forceinline__ void merge_lanes(Softmax<NG>& st) {
  constexpr bool REPL = NG <= 4;
  if constexpr (REPL) {
    // token slots are lane bits 0..2: xor 1, xor 2 within quads, then the
    // other quad of the eight via the half-row mirror
    merge_slots<NG, kDppXor1>(st);
    merge_slots<NG, kDppXor2>(st);
    merge_slots<NG, kDppHalfMirror>(st);
  } else {
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float mo = __shfl_xor(st.m[g], o);
        const float lo = __shfl_xor(st.l[g], o);
        const float mn = __builtin_fmaxf(st.m[g], mo);
        const float ca = __builtin_amdgcn_exp2f(st.m[g] - mn), cb = __builtin_amdgcn_exp2f(mo - mn);
        st.l[g] = st.l[g] * ca + lo * cb;
#pragma unroll
        for (int k = 0; k < 16; ++k) st.acc[g][k] = st.acc[g][k] * ca + __shfl_xor(st.acc[g][k], o) * cb;
        st.m[g] = mn;
      }
    }
  }
}

// The LDS merge of a workgroup's kWaves per-wave states (s_acc, s_m, s_l) into
// partial record rec_idx.
template <int NG>
__device__ __forceinline__ void merge_write(const DecodeArgs& a, int64_t rec_idx, float (*s_acc)[NG][kHead],
                                            float (*s_m)[NG], float (*s_l)[NG]) {
  const int G = a.group;
  __syncthreads();
  const int rec = G * (kHead + 2);
  float* part = a.part + rec_idx * rec;
  for (int i = threadIdx.x; i < G * kHead; i += kWaves * 64) {
    const int g = i / kHead, d = i % kHead;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = __builtin_fmaxf(mx, s_m[w][g]);
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += s_acc[w][g][d] * __builtin_amdgcn_exp2f(s_m[w][g] - mx);
    part[2 * G + i] = v;
  }
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = __builtin_fmaxf(mx, s_m[w][g]);
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum += s_l[w][g] * __builtin_amdgcn_exp2f(s_m[w][g] - mx);
    part[g] = mx;
    part[G + g] = sum;
  }
}

template <int NG>
__device__ __forceinline__ void write_partial(const DecodeArgs& a, Softmax<NG>& st, int64_t rec_idx, int lane,
                                              int wave, float (*s_acc)[NG][kHead]) {
  const int G = a.group;
  constexpr bool REPL = NG <= 4;
  merge_lanes<NG>(st);

  // merge the waves through LDS and write this split's partial
  __shared__ float s_m[kWaves][NG], s_l[kWaves][NG];
  if (token_slot<REPL>(lane) == 0) {  // one lane per column chunk holds the merged state
    const int c = column_chunk<REPL>(lane);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int k = 0; k < 16; ++k) s_acc[wave][g][16 * c + k] = st.acc[g][k];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      s_m[wave][g] = st.m[g];
      s_l[wave][g] = st.l[g];
    }
  }
  merge_write<NG>(a, rec_idx, s_acc, s_m, s_l);
}

// vmcnt <= n, expcnt and lgkmcnt untouched (gfx9 s_waitcnt encoding)
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

// Cache-policy operand of the ring's loads: nt (streamed once, kept out of L2).
constexpr int kDmaNontemporal = 2;

// This lane's two K chunks and two V chunks of a ring slot (LDS byte offsets
// slot + rk0, slot + rk1, slot + rv and slot + rv + 1024), read synchronously.
// Written as one asm block because the compiler, unable to tell which LDS DMA
// wrote which slot, would otherwise wait for every load in flight before any
// LDS read; the caller's explicit vmcnt wait orders the slot's DMA before this.
__device__ __forceinline__ TileLoads ring_read(uint32_t slot, uint32_t rk0, uint32_t rk1, uint32_t rv) {
  const uint32_t a0 = slot + rk0, a1 = slot + rk1, a2 = slot + rv;
  TileLoads c;
  asm volatile(
      "ds_read_b128 %0, %4\n"
      "ds_read_b128 %1, %5\n"
      "ds_read_b128 %2, %6\n"
      "ds_read_b128 %3, %6 offset:1024\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(c.k0), "=&v"(c.k1), "=&v"(c.va), "=&v"(c.vb)
      : "v"(a0), "v"(a1), "v"(a2)
      : "memory");
  return c;
}

// Block sizes that are powers of two >= 16 (a tile lies in one page): each
// wave streams its tiles through a ring of kRing 4 KiB LDS slots filled by
// global_load_lds_dwordx4, so kRing tiles per wave are in flight without
// holding registers (16 waves and 32 tiles per CU at 4 workgroups; a third
// slot per wave, at 3 workgroups per CU, measured 1% slower).
// A slot's four 1 KiB quarters hold the 128-byte head rows of K tokens 0-7,
// K tokens 8-15, V tokens 0-7 and V tokens 8-15.  Each load instruction reads
// eight whole rows, eight lanes per row, so every request covers full cache
// lines; inside a row, 16-byte chunk c of token t sits at 16 * (c ^ (t & 7)),
// and of K token 8 + t at 16 * (c ^ t ^ 1), so that the sixteen lanes reading
// one chunk of sixteen tokens (or of eight V tokens) hit distinct LDS banks.
// The vector-memory counter is waited on explicitly: nothing else in the loop
// uses it.
template <int W, int R = kRing>
struct RingLdsT {
  u32x4 ring[W][R][4][64];
  int32_t pages[kRingPages];
};
using RingLds = RingLdsT<kWaves>;

// ---- P V on the matrix cores ----
//
// Q K^T is computed transposed, S^T = K Q^T (the same four MFMAs with the
// operands swapped): lane l then holds the scores of query head g = l % 16 for
// the four tokens 4 (l / 16) .. +3 of the tile, which is exactly the A operand
// (row g, k = those four tokens) of v_mfma_f32_16x16x16_bf16 for P V.  The B
// operand, V^T (column d, the same four tokens), comes from the ring slot by
// ds_read_b64_tr_b8: in each 16-lane group, result lane i's byte j is byte
// i & 7 of the 8-byte row that source lane 2 j + (i >> 3) addressed.  Source
// lane r of group s addresses token 4 s + ((r >> 1) & 3), bytes 8 (r & 1) ..
// +8 of a 16-byte column chunk, the chunk of block 2 k for r < 8 and of block
// 2 k + 1 otherwise; so one read gives lane l the four tokens of column
// 16 b + l % 16 for two column blocks b (its low and high dword).  P is split
// into bf16 hi + lo (p - hi is exact in fp32 and rounds to bf16 again), so the
// products carry ~16 significant bits of p and the sums are fp32: the same
// accuracy class as fp32 FMAs, with the FMAs off the VALU.  Each lane keeps
// one head's running max and its share of the sum; the MFMA accumulates O
// over all of the wave's tokens, so no lane merge is needed for O.
struct SoftmaxM {
  float m, mth, l;  // head lane % 16: running max (exp2 domain), lazy threshold, this lane's part of the sum
  f32x4 o[8];       // O[4 (lane / 16) + r][16 b + lane % 16] = o[b][r]
};

__device__ __forceinline__ void softmax_init(SoftmaxM& st) {
  st.m = kNegBig;
  st.mth = kNegBig + kLazy;
  st.l = 0.0f;
#pragma unroll
  for (int b = 0; b < 8; ++b) st.o[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// Byte offsets (from a ring slot) of this lane's four transposed-read rows:
// V token 4 s + ((r >> 1) & 3), chunk 2 k (r < 8) or 2 k + 1, half r & 1,
// with the slot's XOR swizzle (chunk c of token t at 16 (c ^ (t & 7))).
__device__ __forceinline__ void pv_offsets(int lane, uint32_t (&off)[4]) {
  const int r = lane & 15, s = lane >> 4;
  const int tok = 4 * s + ((r >> 1) & 3);
  const uint32_t row = uint32_t(2048 + 1024 * (tok >> 3) + 128 * (tok & 7) + 8 * (r & 1));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = 2 * k + (r >= 8 ? 1 : 0);
    off[k] = row + uint32_t(16 * (c ^ (tok & 7)));
  }
}

// K (as ring_read) and the eight V^T operand words of a slot, read
// synchronously in one asm block (see ring_read for why).
__device__ __forceinline__ void ring_read_pv(uint32_t slot, uint32_t rk0, uint32_t rk1, const uint32_t (&off)[4],
                                             u32x4& k0, u32x4& k1, uint32_t (&vw)[8]) {
  i32x2 t0, t1, t2, t3;
  asm volatile(
      "ds_read_b128 %0, %6\n"
      "ds_read_b128 %1, %7\n"
      "ds_read_b64_tr_b8 %2, %8\n"
      "ds_read_b64_tr_b8 %3, %9\n"
      "ds_read_b64_tr_b8 %4, %10\n"
      "ds_read_b64_tr_b8 %5, %11\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(k0), "=&v"(k1), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "v"(slot + rk0), "v"(slot + rk1), "v"(slot + off[0]), "v"(slot + off[1]), "v"(slot + off[2]),
        "v"(slot + off[3])
      : "memory");
  vw[0] = uint32_t(t0[0]);
  vw[1] = uint32_t(t0[1]);
  vw[2] = uint32_t(t1[0]);
  vw[3] = uint32_t(t1[1]);
  vw[4] = uint32_t(t2[0]);
  vw[5] = uint32_t(t2[1]);
  vw[6] = uint32_t(t3[0]);
  vw[7] = uint32_t(t3[1]);
}

// One 16-token tile of one wave on the matrix cores.  vw: V^T words (byte j =
// token 4 (lane / 16) + j of column 16 b + lane % 16), zero for a missing page;
// rows 0 .. G-1 are the group's (query token, query head) pairs.
//
// MASKED: a tile that reaches t_end or the causal band; this lane's row then
// sees keys below min(t_end, row_lim).  Every other tile is whole and visible
// to every row.
template <bool MASKED, class Consumed>
__device__ __forceinline__ void attend_step_pv(SoftmaxM& st, const u32x4& k0, const u32x4& k1,
                                               const uint32_t (&vw)[8], const bf16x8 qop[4], float sl, int t0,
                                               int t_end, int G, int lane, int row_lim, const Consumed& consumed) {
  f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_to_bf16(k0[0], k0[1]), qop[0], sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_to_bf16(k0[2], k0[3]), qop[1], sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_to_bf16(k1[0], k1[1]), qop[2], sc, 0, 0, 0);
  sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_to_bf16(k1[2], k1[3]), qop[3], sc, 0, 0, 0);
  consumed();

  const int g = lane & 15, tq = 4 * (lane >> 4);
  float s4[4];
  const int lim = MASKED ? min(t_end, row_lim) : 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool ok = g < G && (!MASKED || t0 + tq + r < lim);
    s4[r] = ok ? sc[r] * sl : -__builtin_inff();
  }
  float mx = __builtin_fmaxf(__builtin_fmaxf(s4[0], s4[1]), __builtin_fmaxf(s4[2], s4[3]));
  mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
  mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));  // head g's tile max, in its four lanes
  if (__any(mx > st.mth)) {
    const float mn = __builtin_fmaxf(st.m, mx);
    const float c = __builtin_amdgcn_exp2f(st.m - mn);
    st.l *= c;
    st.m = mn;
    st.mth = mn + kLazy;
    // O row 4 (lane / 16) + r takes its head's factor from that head's lane
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cr = bperm(tq + r, c);
#pragma unroll
      for (int b = 0; b < 8; ++b) st.o[b][r] *= cr;
    }
  }
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(s4[r] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  const bf16x4 hi = {(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3]};
  const bf16x4 lo = {(__bf16)(p[0] - (float)hi[0]), (__bf16)(p[1] - (float)hi[1]), (__bf16)(p[2] - (float)hi[2]),
                     (__bf16)(p[3] - (float)hi[3])};
  uint32_t vmask = 0xFFFFFFFFu;
  if constexpr (MASKED) {
    // tokens at or past t_end may hold anything (a NaN would survive p = 0)
    const int n_ok = t_end - (t0 + tq);
    vmask = n_ok >= 4 ? 0xFFFFFFFFu : n_ok <= 0 ? 0u : (0xFFFFFFFFu >> (32 - 8 * n_ok));
  }
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint32_t w = vw[b] & vmask;
    const bf16x2 v01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const bf16x2 v23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    const bf16x4 vb = {v01[0], v01[1], v23[0], v23[1]};
    st.o[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, hi), __builtin_bit_cast(s16x4, vb),
                                                        st.o[b], 0, 0, 0);
    st.o[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, lo), __builtin_bit_cast(s16x4, vb),
                                                        st.o[b], 0, 0, 0);
  }
}

// The wave's record of a P V-on-MFMA state: head g's sum over its four lanes,
// then either stored directly (record at `part`) or stashed in LDS for a
// cross-wave merge.
__device__ __forceinline__ void finish_sum(SoftmaxM& st) {
  st.l += __shfl_xor(st.l, 16);
  st.l += __shfl_xor(st.l, 32);
}

__device__ __forceinline__ void write_record_pv(const SoftmaxM& st, float* part, int G, int lane) {
  const int g = lane & 15, q = lane >> 4;
  if (q == 0 && g < G) {
    part[g] = st.m;
    part[G + g] = st.l;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int gr = 4 * q + r;
    if (gr < G) {
#pragma unroll
      for (int b = 0; b < 8; ++b) part[2 * G + gr * kHead + 16 * b + g] = st.o[b][r];
    }
  }
}

template <int NG>
__device__ __forceinline__ void stash_pv(const SoftmaxM& st, float (*s_acc)[NG][kHead], float (*s_m)[NG],
                                         float (*s_l)[NG], int wave, int lane) {
  const int g = lane & 15, q = lane >> 4;
  if (q == 0 && g < NG) {
    s_m[wave][g] = st.m;
    s_l[wave][g] = st.l;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int gr = 4 * q + r;
    if (gr < NG) {
#pragma unroll
      for (int b = 0; b < 8; ++b) s_acc[wave][gr][16 * b + g] = st.o[b][r];
    }
  }
}

template <int NG>
__device__ __forceinline__ void write_partial(const DecodeArgs& a, SoftmaxM& st, int64_t rec_idx, int lane, int wave,
                                              float (*s_acc)[NG][kHead]) {
  finish_sum(st);
  __shared__ float s_m[kWaves][NG], s_l[kWaves][NG];
  stash_pv<NG>(st, s_acc, s_m, s_l, wave, lane);
  merge_write<NG>(a, rec_idx, s_acc, s_m, s_l);
}

// s_waitcnt vmcnt(n) for a run-time n < 16 (the immediate must be a constant)
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4)); break;
    case 8: __builtin_amdgcn_s_waitcnt(vmcnt_imm(8)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(12)); break;
  }
}

// Tokens [t_begin, t_end) of (sequence b, kv head h) into the running softmax
// st of this wave, which takes tiles t_begin + 16 phase + 16 P j (phase < P).
// t_begin is a multiple of 16 and the range spans at most kRingPages pages.
// Called by all W waves of the workgroup with the same sequence and range (the
// heads may differ): it stages the range's page ids behind a barrier.
// `overlap` runs while the page-id loads are in flight (a new head's query
// loads go there, so that both cost one memory latency).
//
// GEN selects the addressing.  Without it the block size is a power of two >=
// 16, so a tile lies in one page: the page id and row base are wave-uniform,
// each lane adds a fixed 32-bit offset, and a missing page zeroes the slot.
// With it (any other block size, or rows too far apart for 32-bit offsets)
// the rows of a tile may come from different pages: each lane keeps the page
// index and row of its two load rows, advanced by the tile stride, and
// addresses them in 64 bits; a row on a missing page (or past t_end) loads row
// 0 of page 0 instead, and a per-slot mask of the tile's 16 tokens (from two
// ballots at issue) zeroes those tokens' K and V when the slot is read.
template <int NG, int W, int P, int R, bool GEN, class ST, class Overlap>
__device__ __forceinline__ void ring_attend(const DecodeArgs& a, ST& st, const bf16x8 (&qop)[4],
                                            const float& sl, int b, int h, int t_begin, int t_end, int len, int lane,
                                            int wave, int phase, RingLdsT<W, R>& lds, const Overlap& overlap) {
  static_assert(R >= 2 && R <= 4, "ring of 2 to 4 tiles per wave");
  constexpr int kIdsPerThread = kRingPages / (W * 64);
  static_assert(kRingPages % (W * 64) == 0, "page ids are staged a whole number per thread");
  const int32_t* bt_row = a.block_table + b * a.bt_stride;
  const int first = GEN ? page_index(a, t_begin) : t_begin >> a.bs_shift;
  const int n_ids = (GEN ? page_index(a, t_end - 1) : (t_end - 1) >> a.bs_shift) - first + 1;
  __syncthreads();  // the previous range's readers of pages and ring are done
  int32_t ids[kIdsPerThread];
#pragma unroll
  for (int k = 0; k < kIdsPerThread; ++k) {
    const int i = int(threadIdx.x) + k * W * 64;
    ids[k] = i < n_ids ? checked_page(a, bt_row, first + i) : -1;
  }
  overlap();
#pragma unroll
  for (int k = 0; k < kIdsPerThread; ++k) {
    const int i = int(threadIdx.x) + k * W * 64;
    if (i < n_ids) lds.pages[i] = ids[k];
  }
  __syncthreads();
  u32x4(*ring)[4][64] = lds.ring[wave];

  // load side: lane l fetches the chunk stored at position l & 7 of row l >> 3
  const int drow = lane >> 3, dchunk = (lane & 7) ^ (lane >> 3);
  const uint32_t off_k = uint32_t(drow * a.k_row + 16 * dchunk);
  const uint32_t off_k8 = uint32_t((8 + drow) * a.k_row + 16 * (dchunk ^ 1));
  const uint32_t off_v = uint32_t(drow * a.v_row + 16 * dchunk);
  const uint32_t off_v8 = uint32_t(off_v + 8 * a.v_row);
  // read side: K bytes 32 * (l >> 4) .. + 32 of token l & 15 (the MFMA's B
  // operand), V chunk column_chunk(l) of tokens token_slot(l) and + 8
  const int kt = lane & 15, kc = 2 * (lane >> 4), kx = (kt & 7) ^ (kt >> 3);
  const uint32_t rk0 = uint32_t(1024 * (kt >> 3) + 128 * (kt & 7) + 16 * (kc ^ kx));
  const uint32_t rk1 = uint32_t(1024 * (kt >> 3) + 128 * (kt & 7) + 16 * ((kc + 1) ^ kx));
  const int vt = token_slot<(NG <= 4)>(lane), vc = column_chunk<(NG <= 4)>(lane);
  const uint32_t rv = uint32_t(2048 + 128 * vt + 16 * (vc ^ vt));
  const int stride = kTile * P;
  const int t_first = t_begin + phase * kTile;
  const int n_tiles = t_first < t_end ? (t_end - t_first + stride - 1) / stride : 0;

  // GEN: page index and row of this lane's load rows (tokens t0 + drow and
  // t0 + drow + 8 of the next tile to issue), and the tile stride in pages
  // and rows
  int pia = 0, ra = 0, pib = 0, rb = 0, sq = 0, sr = 0;
  uint64_t tok_ok = 0;  // GEN: bits 16 s .. 16 s + 15: tokens of slot s on real pages
  if constexpr (GEN) {
    const int bs = a.block_size;
    const int ta = t_first + drow;
    pia = page_index(a, ta);
    ra = ta - pia * bs;
    pib = page_index(a, ta + 8);
    rb = ta + 8 - pib * bs;
    sq = page_index(a, stride);
    sr = stride - sq * bs;
  }

  // start the loads of tile j into its slot; a missing page reads page 0 (in
  // bounds) and is zeroed when consumed.  Before a new tile goes out, the
  // loads still in flight land: the waves of a workgroup, which read the same
  // token rows, then stay in step.  Config 2's decode: 225 us; two tiles in
  // flight per wave 230; a three-slot ring with one or two in flight 227 and
  // 235
  uint32_t valid = 0;  // bit j % R: slot holds a tile on a real page
  auto issue = [&](int j) {
    const int t0 = t_first + j * stride;
    const int slot = j % R;
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    if constexpr (GEN) {
      const int ta = t0 + drow;
      const int32_t ida = ta < t_end ? lds.pages[pia - first] : -1;
      const int32_t idb = ta + 8 < t_end ? lds.pages[pib - first] : -1;
      // every lane of a row agrees, so bit 8 r of a ballot is row r's
      const uint64_t ba = __ballot(ida >= 0) & 0x0101010101010101ull;
      const uint64_t bb = __ballot(idb >= 0) & 0x0101010101010101ull;
      const uint64_t m16 = ((ba * 0x0102040810204080ull) >> 56) | (((bb * 0x0102040810204080ull) >> 56) << 8);
      tok_ok = (tok_ok & ~(0xFFFFull << (16 * slot))) | (m16 << (16 * slot));
      const int64_t pa = ida >= 0 ? ida : 0, rwa = ida >= 0 ? ra : 0;
      const int64_t pb = idb >= 0 ? idb : 0, rwb = idb >= 0 ? rb : 0;
      const uint8_t* ka = a.k + pa * a.k_blk + rwa * a.k_row + int64_t(h) * a.k_head;
      const uint8_t* kb = a.k + pb * a.k_blk + rwb * a.k_row + int64_t(h) * a.k_head;
      const uint8_t* va = a.v + pa * a.v_blk + rwa * a.v_row + int64_t(h) * a.v_head;
      const uint8_t* vb = a.v + pb * a.v_blk + rwb * a.v_row + int64_t(h) * a.v_head;
      __builtin_amdgcn_global_load_lds((gvoid*)(ka + 16 * dchunk), (lvoid*)&ring[slot][0][0], 16, 0, kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(kb + 16 * (dchunk ^ 1)), (lvoid*)&ring[slot][1][0], 16, 0,
                                       kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(va + 16 * dchunk), (lvoid*)&ring[slot][2][0], 16, 0, kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(vb + 16 * dchunk), (lvoid*)&ring[slot][3][0], 16, 0, kDmaNontemporal);
      pia += sq;
      ra += sr;
      if (ra >= a.block_size) {
        ra -= a.block_size;
        ++pia;
      }
      pib += sq;
      rb += sr;
      if (rb >= a.block_size) {
        rb -= a.block_size;
        ++pib;
      }
    } else {
      const int32_t raw = __builtin_amdgcn_readfirstlane(lds.pages[(t0 >> a.bs_shift) - first]);
      valid = raw >= 0 ? (valid | (1u << slot)) : (valid & ~(1u << slot));
      const int64_t pid = raw >= 0 ? raw : 0;
      const int64_t row0 = t0 & (a.block_size - 1);
      const uint8_t* kb = a.k + pid * a.k_blk + row0 * a.k_row + int64_t(h) * a.k_head;
      const uint8_t* vb = a.v + pid * a.v_blk + row0 * a.v_row + int64_t(h) * a.v_head;
      __builtin_amdgcn_global_load_lds((gvoid*)(kb + off_k), (lvoid*)&ring[slot][0][0], 16, 0, kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(kb + off_k8), (lvoid*)&ring[slot][1][0], 16, 0, kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(vb + off_v), (lvoid*)&ring[slot][2][0], 16, 0, kDmaNontemporal);
      __builtin_amdgcn_global_load_lds((gvoid*)(vb + off_v8), (lvoid*)&ring[slot][3][0], 16, 0, kDmaNontemporal);
    }
  };
  // GEN: the 16-token mask of a slot
  auto slot_tokens = [&](int slot) { return uint32_t(tok_ok >> (16 * slot)) & 0xFFFFu; };
  auto fetch = [&](int j) {
    // tiles issued after j: min(R - 1, n_tiles - 1 - j), four loads each
    if (j + R - 1 < n_tiles) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * (R - 1)));
    else wait_vmcnt(4 * (n_tiles - 1 - j));
    const int slot = j % R;
    TileLoads c = ring_read((uint32_t)(size_t)(lvoid*)&ring[slot][0][0], rk0, rk1, rv);
    if constexpr (GEN) {
      const uint32_t m = slot_tokens(slot);
      if (!((m >> kt) & 1u)) c.k0 = c.k1 = u32x4(0);
      if (!((m >> vt) & 1u)) c.va = u32x4(0);
      if (!((m >> (vt + 8)) & 1u)) c.vb = u32x4(0);
    } else {
      if (!((valid >> slot) & 1u)) c.k0 = c.k1 = c.va = c.vb = u32x4(0);
    }
    return c;
  };
  for (int j = 0; j < R && j < n_tiles; ++j) issue(j);
  if constexpr (std::is_same_v<ST, SoftmaxM>) {
    uint32_t off[4];
    pv_offsets(lane, off);
    const int G = a.group;
    struct PvTile {
      u32x4 k0, k1;
      uint32_t vw[8];
    };
    auto fetch_pv = [&](int j) {
      if (j + R - 1 < n_tiles) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * (R - 1)));
      else wait_vmcnt(4 * (n_tiles - 1 - j));
      const int slot = j % R;
      PvTile c;
      ring_read_pv((uint32_t)(size_t)(lvoid*)&ring[slot][0][0], rk0, rk1, off, c.k0, c.k1, c.vw);
      if constexpr (GEN) {
        // K: token lane & 15; V^T word byte i: token 4 (lane / 16) + i
        const uint32_t m = slot_tokens(slot);
        if (!((m >> kt) & 1u)) c.k0 = c.k1 = u32x4(0);
        const uint32_t nib = (m >> (4 * (lane >> 4))) & 0xFu;
        const uint32_t bytes = ((nib * 0x00204081u) & 0x01010101u) * 0xFFu;
#pragma unroll
        for (int b = 0; b < 8; ++b) c.vw[b] &= bytes;
      } else if (!((valid >> slot) & 1u)) {
        c.k0 = c.k1 = u32x4(0);
#pragma unroll
        for (int b = 0; b < 8; ++b) c.vw[b] = 0u;
      }
      return c;
    };
    // query token i of n sees keys below causal_lo + i, causal_lo = len - n + 1
    // when causal (FA's bottom-right alignment), else every key: row_lim
    const int causal_lo = __builtin_amdgcn_readfirstlane(a.causal ? len - max(q_count(a, b), 1) + 1 : len);
    const int qrow = lane & 15;
    const int row_lim = causal_lo + (a.causal && qrow < G ? qrow / a.heads : 0);
    if (n_tiles > 0) {
      // tiles j >= j_mask reach t_end or causal_lo and mask per row: the last
      // one, and with several query tokens and a one-tile stride possibly the
      // one before (causal_lo > len - 16); the loop over the others has no test
      const int lo = causal_lo - kTile - t_first;
      const int j_mask = min(n_tiles - 1, lo < 0 ? 0 : lo / stride + 1);
      int j = 0;
      for (; j < j_mask; ++j) {
        PvTile c = fetch_pv(j);
        attend_step_pv<false>(st, c.k0, c.k1, c.vw, qop, sl, t_first + j * stride, t_end, G, lane, row_lim, [&] {
          if (j + R < n_tiles) issue(j + R);
        });
      }
      for (; j < n_tiles; ++j) {
        PvTile c = fetch_pv(j);
        attend_step_pv<true>(st, c.k0, c.k1, c.vw, qop, sl, t_first + j * stride, t_end, G, lane, row_lim, [&] {
          if (j + R < n_tiles) issue(j + R);
        });
      }
    }
  } else {
    if (n_tiles > 0) {
      int j = 0;
      for (; j + 1 < n_tiles; ++j) {
        TileLoads c = fetch(j);
        attend_step<NG, false>(st, c, qop, sl, t_first + j * stride, t_end, lane, [&] {
          if (j + R < n_tiles) issue(j + R);
        });
      }
      TileLoads c = fetch(j);
      attend_step<NG, true>(st, c, qop, sl, t_first + j * stride, t_end, lane, [] {});
    }
  }
}

// Tokens per page-id staging piece of a range: whole multiples of `align`
// (the tile stride of every phase), spanning at most kRingPages pages from
// any 16-aligned start.
__device__ __forceinline__ int staging_piece(const DecodeArgs& a, int align) {
  const int64_t tokens = a.bs_shift >= 0 ? int64_t(kRingPages - 1) << a.bs_shift
                                         : int64_t(kRingPages - 1) * a.block_size;
  return int(std::min<int64_t>(tokens, INT32_MAX / 2)) & ~(align - 1);
}

template <int NG>
__device__ __forceinline__ void softmax_init(Softmax<NG>& st) {
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    st.m[g] = kNegBig;
    st.mth[g] = kNegBig + kLazy;
    st.l[g] = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) st.acc[g][k] = 0.0f;
  }
}

// Query operands and the score scale of (sequence b, kv head h).  REPL: rows
// replicated in the four row quarters (the VALU P V path for groups of at
// most 4 heads); otherwise row i is query head i.
template <int NG, bool REPL = (NG <= 4)>
__device__ __forceinline__ float load_head(const DecodeArgs& a, int q_dtype, int b, int h, int lane, bf16x8 qop[4]) {
  const float qd = descale(a.qd, a.qd_b, a.qd_h, b, h);
  const float kd = descale(a.kd, a.kd_b, a.kd_h, b, h);
  uint32_t qw[8];
  load_query<REPL>(a, q_dtype, b, h, qd, lane, qw);
  qop[0] = e4m3x8_to_bf16(qw[0], qw[1]);
  qop[1] = e4m3x8_to_bf16(qw[2], qw[3]);
  qop[2] = e4m3x8_to_bf16(qw[4], qw[5]);
  qop[3] = e4m3x8_to_bf16(qw[6], qw[7]);
  return a.scale_log2 * qd * kd;
}

// P V on the matrix cores (PSK_PV_MFMA=0 builds the VALU P V of attend_step
// instead, in fp32, for comparison).
#ifndef PSK_PV_MFMA
#define PSK_PV_MFMA 1
#endif
constexpr bool kPvMfma = PSK_PV_MFMA != 0;
template <int NG>
using BalancedState = std::conditional_t<kPvMfma, SoftmaxM, Softmax<NG>>;

// One workgroup per (split, kv head, sequence) (an explicit num_splits).
template <int NG, bool GEN>
__global__ void __launch_bounds__(kWaves * 64) decode_partial_ring_kernel(DecodeArgs a, int q_dtype) {
  // split s of sequence b sits at blockIdx.x = (s + b) % max_splits: workgroups
  // go round-robin to the 8 XCDs by blockIdx.x (max_splits is the fastest grid
  // dimension), so the first splits of short sequences spread over all of them
  const int h = blockIdx.y, b = blockIdx.z;
  const int s = int((blockIdx.x + unsigned(a.max_splits) - unsigned(b % a.max_splits)) % unsigned(a.max_splits));
  const int len = a.seq_lens[b];
  const int t_begin = s * a.split;
  if (t_begin >= len || s >= a.max_splits) return;  // uniform over the workgroup
  const int t_end = min(len, t_begin + a.split);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  __shared__ RingLds lds;
  static_assert(sizeof(lds.ring) >= sizeof(float) * kWaves * NG * kHead, "the ring doubles as the merge buffer");
  bf16x8 qop[4];
  float sl = 0.0f;
  BalancedState<NG> st;
  softmax_init(st);
  // the split in pieces of at most kRingPages pages (one piece unless the pages are small)
  const int piece = staging_piece(a, kTile * kWaves);
  for (int t0 = t_begin; t0 < t_end; t0 += piece) {
    const bool head = t0 == t_begin;
    ring_attend<NG, kWaves, kWaves, kRing, GEN>(a, st, qop, sl, b, h, t0, min(t_end, t0 + piece), len, lane, wave,
                                                wave, lds, [&] {
      if (head) sl = load_head<NG, !kPvMfma && (NG <= 4)>(a, q_dtype, b, h, lane, qop);
    });
  }
  __syncthreads();  // every wave is done with the ring: it becomes the merge buffer
  write_partial<NG>(a, st, (int64_t(b) * a.num_kv_heads + h) * a.max_splits + s, lane, wave,
                    reinterpret_cast<float(*)[NG][kHead]>(&lds.ring[0][0][0][0]));
}

// Balanced schedule.  Per kv head the work is a list of units: for each
// sequence b with tokens, seq_units units that carry no work (the cost of
// starting a sequence) and then its 16-token tiles t, ceil(len_b / 16) of
// them; T units in all.  Run j of head h takes head h's units
// [T j / M, T (j+1) / M), M = min(grid / Hkv, T), whatever sequences they
// belong to: every workgroup gets the same cost in tiles and sequence starts,
// the grid (one workgroup per resident slot) ends together,
// and the Hkv workgroups of one j walk the same tokens of the same pages at
// the same time (a token's kv heads share its cache rows).  Workgroup
// j * Hkv + h runs (h, j): the heads of one run are dispatched together.  Each maximal run
// of one sequence inside the range gives one partial record, at index
// (b + j) * Hkv + h: the records of one (b, h) come from consecutive j, Hkv
// apart.  Workgroup 0 also stores the units prefix (prefix[b] = units before
// b) after the records for the combine.
__device__ __forceinline__ int tiles_of(int len) { return len > 0 ? (len + kTile - 1) / kTile : 0; }

// Units of sequence b in the balanced schedule: its tiles, after a.seq_units
// units that carry no work and stand for the fixed cost of starting a
// sequence (page-id staging, query loads, the partial record), so that a run
// over many short sequences takes fewer tiles.
__device__ __forceinline__ int units_of(const DecodeArgs& a, int len) {
  return len > 0 ? tiles_of(len) + a.seq_units : 0;
}

// Units prefix of the batch in LDS (pref[b] = units before sequence b,
// pref[num_seqs] = all units), by the NT threads of the workgroup; returns the
// total.  `store` also writes it to a.prefix for the combine; `lens`, when
// given, receives a copy of the sequence lengths.
template <int NT>
__device__ __forceinline__ int64_t scan_tiles(const DecodeArgs& a, int num_seqs, int32_t* pref, int32_t* s_scan,
                                              bool store, int32_t* lens = nullptr) {
  const int tid = threadIdx.x;
  const int chunk = (num_seqs + NT - 1) / NT;
  int sum = 0;
  for (int i = 0; i < chunk; ++i) {
    const int b = tid * chunk + i;
    if (b < num_seqs) {
      const int len = a.seq_lens[b];
      if (lens) lens[b] = len;
      sum += units_of(a, len);
    }
  }
  s_scan[tid] = sum;
  __syncthreads();
  for (int o = 1; o < NT; o <<= 1) {
    const int v = tid >= o ? s_scan[tid - o] : 0;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  int run = tid > 0 ? s_scan[tid - 1] : 0;
  for (int i = 0; i < chunk; ++i) {
    const int b = tid * chunk + i;
    if (b < num_seqs) {
      pref[b] = run;
      run += units_of(a, lens ? lens[b] : a.seq_lens[b]);
    }
  }
  if (tid == NT - 1) pref[num_seqs] = s_scan[NT - 1];
  __syncthreads();
  if (store) {
    for (int i = tid; i <= num_seqs; i += NT) a.prefix[i] = pref[i];
  }
  return pref[num_seqs];
}

// The sequence b that owns unit u (the last with pref[b] <= u: sequences
// without units share their successor's prefix) and the tile t of b that unit
// u stands for, negative inside b's leading units.
__device__ __forceinline__ void seek_unit(const int32_t* pref, int num_seqs, int seq_units, int64_t u, int& b,
                                          int& t) {
  int lo = 0, hi = num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pref[mid] <= u) lo = mid; else hi = mid - 1;
  }
  b = lo;
  t = int(u - pref[b]) - seq_units;
}

// Three waves per SIMD: left to itself the compiler keeps the MFMA accumulators in
// AGPRs, which puts the general-page variant at 141 VGPRs + 36 AGPRs and two waves
// per SIMD; asked for three it fits every variant in 143 VGPRs without spilling.
template <int NG, bool GEN>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(3)))
decode_partial_stream_kernel(DecodeArgs a, int q_dtype, int num_seqs) {
  const int w = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int Hkv = a.num_kv_heads;
  __shared__ RingLds lds;
  static_assert(sizeof(lds.ring) >= sizeof(float) * kWaves * NG * kHead, "the ring doubles as the merge buffer");
  static_assert(sizeof(lds.ring) / sizeof(int32_t) > kStreamMaxSeqs, "the ring holds the units prefix");

  // units prefix over the sequences, scanned in the ring (free until the first tile)
  int32_t* pref = reinterpret_cast<int32_t*>(&lds.ring[0][0][0][0]);
  __shared__ int32_t s_scan[kWaves * 64];
  const int64_t T = scan_tiles<kWaves * 64>(a, num_seqs, pref, s_scan, w == 0);
  // no more runs than units, so that no range is empty and the records of one
  // (b, h) stay consecutive; the other workgroups leave
  const int h = w % Hkv, j = w / Hkv;
  const int64_t M = min<int64_t>(gridDim.x / Hkv, T);
  if (j >= M) return;  // uniform over the workgroup
  int64_t u = T * j / M;
  const int64_t u_end = T * (j + 1) / M;
  int b, t;
  seek_unit(pref, num_seqs, a.seq_units, u, b, t);
  // ring_attend's first barrier orders these prefix reads before the ring is refilled

  const int piece = staging_piece(a, kTile * kWaves);
  while (u < u_end && b < num_seqs) {
    if (t < 0) {  // leading units of b: no work
      const int skip = int(min<int64_t>(-t, u_end - u));
      u += skip;
      t += skip;
      if (u >= u_end) break;
    }
    const int len = a.seq_lens[b];
    const int tb = tiles_of(len);
    const int n = int(min<int64_t>(tb - t, u_end - u));
    bf16x8 qop[4];
    float sl = 0.0f;
    BalancedState<NG> st;
    softmax_init(st);
    const int t_end = min(len, (t + n) * kTile);
    for (int t0 = t * kTile; t0 < t_end; t0 += piece) {
      const bool head = t0 == t * kTile;
      ring_attend<NG, kWaves, kWaves, kRing, GEN>(a, st, qop, sl, b, h, t0, min(t_end, t0 + piece), len, lane, wave,
                                                  wave, lds, [&] {
        if (head) sl = load_head<NG, !kPvMfma && (NG <= 4)>(a, q_dtype, b, h, lane, qop);
      });
    }
    __syncthreads();  // every wave is done with the ring: it becomes the merge buffer
    write_partial<NG>(a, st, (int64_t(b) + j) * Hkv + h, lane, wave,
                      reinterpret_cast<float(*)[NG][kHead]>(&lds.ring[0][0][0][0]));
    u += n;
    t += n;
    if (t == tb) {
      t = -a.seq_units;
      do ++b; while (b < num_seqs && a.seq_lens[b] <= 0);
    }
  }
}

// Head-parallel balanced schedule.  The same units and runs as
// decode_partial_stream_kernel, but one workgroup of kHeadWaves waves takes a
// run for HG kv heads at once: wave w serves head hg * HG + w % HG and tile
// phase w / HG (P = kHeadWaves / HG phases).  With HG = 8 every wave walks
// all of the run's tiles for its own head, so at any moment one CU requests
// whole 1 KiB token rows (all heads' 128-byte slices of a token) instead of
// each of eight workgroups on eight XCDs requesting its own slice: a
// read-only probe of config 2's pages streams 6.9 TB/s that way against 5.9
// for head slices.  Workgroup j * NHG + hg serves run j of head group hg
// (NHG = Hkv / HG); records and the units prefix are laid out as in the
// per-head balanced schedule, so the same combine reads them.
constexpr int kHeadWaves = 8;
// LDS tile slots per wave.  At one workgroup per CU deeper rings cost no
// occupancy, but measured slower on config 2: 227 us at three against 225.
constexpr int kHeadRing = 2;


// Merge this wave's token slots and, with P phases per head, the P waves of
// each head through LDS; write head h's partial record rec_idx.
template <int NG, int HG, int P>
__device__ __forceinline__ void write_partial_heads(const DecodeArgs& a, Softmax<NG>& st, int64_t rec_idx, int lane,
                                                    int wave, float (*s_acc)[NG][kHead], float (*s_m)[NG],
                                                    float (*s_l)[NG]) {
  const int G = a.group;
  constexpr bool REPL = NG <= 4;
  merge_lanes<NG>(st);
  float* part = a.part + rec_idx * (G * (kHead + 2));
  if constexpr (P == 1) {
    if (token_slot<REPL>(lane) == 0) {
      const int c = column_chunk<REPL>(lane);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < G) {
#pragma unroll
          for (int k = 0; k < 16; ++k) part[2 * G + g * kHead + 16 * c + k] = st.acc[g][k];
        }
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < G) {
          part[g] = st.m[g];
          part[G + g] = st.l[g];
        }
      }
    }
  } else {
    if (token_slot<REPL>(lane) == 0) {
      const int c = column_chunk<REPL>(lane);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int k = 0; k < 16; ++k) s_acc[wave][g][16 * c + k] = st.acc[g][k];
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        s_m[wave][g] = st.m[g];
        s_l[wave][g] = st.l[g];
      }
    }
    __syncthreads();
    if (wave < HG) {  // phase 0 of head `wave` writes the merged record
      for (int i = lane; i < G * kHead; i += 64) {
        const int g = i / kHead, d = i % kHead;
        float mx = s_m[wave][g];
#pragma unroll
        for (int p = 1; p < P; ++p) mx = __builtin_fmaxf(mx, s_m[wave + HG * p][g]);
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) v += s_acc[wave + HG * p][g][d] * __builtin_amdgcn_exp2f(s_m[wave + HG * p][g] - mx);
        part[2 * G + i] = v;
      }
      if (lane < G) {
        const int g = lane;
        float mx = s_m[wave][g];
#pragma unroll
        for (int p = 1; p < P; ++p) mx = __builtin_fmaxf(mx, s_m[wave + HG * p][g]);
        float sum = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) sum += s_l[wave + HG * p][g] * __builtin_amdgcn_exp2f(s_m[wave + HG * p][g] - mx);
        part[g] = mx;
        part[G + g] = sum;
      }
    }
  }
}

template <int NG, int HG, int P>
__device__ __forceinline__ void write_partial_heads(const DecodeArgs& a, SoftmaxM& st, int64_t rec_idx, int lane,
                                                    int wave, float (*s_acc)[NG][kHead], float (*s_m)[NG],
                                                    float (*s_l)[NG]) {
  const int G = a.group;
  finish_sum(st);
  float* part = a.part + rec_idx * (G * (kHead + 2));
  if constexpr (P == 1) {
    write_record_pv(st, part, G, lane);
  } else {
    stash_pv<NG>(st, s_acc, s_m, s_l, wave, lane);
    __syncthreads();
    if (wave < HG) {  // phase 0 of head `wave` writes the merged record
      for (int i = lane; i < G * kHead; i += 64) {
        const int g = i / kHead, d = i % kHead;
        float mx = s_m[wave][g];
#pragma unroll
        for (int p = 1; p < P; ++p) mx = __builtin_fmaxf(mx, s_m[wave + HG * p][g]);
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) v += s_acc[wave + HG * p][g][d] * __builtin_amdgcn_exp2f(s_m[wave + HG * p][g] - mx);
        part[2 * G + i] = v;
      }
      if (lane < G) {
        const int g = lane;
        float mx = s_m[wave][g];
#pragma unroll
        for (int p = 1; p < P; ++p) mx = __builtin_fmaxf(mx, s_m[wave + HG * p][g]);
        float sum = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) sum += s_l[wave + HG * p][g] * __builtin_amdgcn_exp2f(s_m[wave + HG * p][g] - mx);
        part[g] = mx;
        part[G + g] = sum;
      }
    }
  }
}

template <int NG, int HG, bool GEN>
__global__ void __launch_bounds__(kHeadWaves * 64) decode_partial_heads_kernel(DecodeArgs a, int q_dtype,
                                                                              int num_seqs) {
  constexpr int W = kHeadWaves;
  constexpr int P = W / HG;
  const int w = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int Hkv = a.num_kv_heads;
  const int NHG = Hkv / HG;
  __shared__ RingLdsT<W, kHeadRing> lds;
  __shared__ float s_m[W][NG], s_l[W][NG];
  static_assert(sizeof(lds.ring) >= sizeof(float) * W * NG * kHead, "the ring doubles as the merge buffer");

  // units prefix and lengths of the sequences, kept in LDS for the whole run
  __shared__ int32_t s_pref[kStreamMaxSeqs + 1], s_len[kStreamMaxSeqs];
  __shared__ int32_t s_scan[W * 64];
  const int64_t T = scan_tiles<W * 64>(a, num_seqs, s_pref, s_scan, w == 0, s_len);
  const int hg = w % NHG, j = w / NHG;
  const int h = hg * HG + wave % HG, phase = wave / HG;
  const int64_t M = min<int64_t>(gridDim.x / NHG, T);
  if (j >= M) return;  // uniform over the workgroup
  int64_t u = T * j / M;
  const int64_t u_end = T * (j + 1) / M;
  int b, t;
  seek_unit(s_pref, num_seqs, a.seq_units, u, b, t);

  // page-id staging pieces: whole multiples of every phase stride
  const int piece = staging_piece(a, kTile * W);
  while (u < u_end && b < num_seqs) {
    if (t < 0) {  // leading units of b: no work
      const int skip = int(min<int64_t>(-t, u_end - u));
      u += skip;
      t += skip;
      if (u >= u_end) break;
    }
    const int len = s_len[b];
    const int tb = tiles_of(len);
    const int n = int(min<int64_t>(tb - t, u_end - u));
    bf16x8 qop[4];
    float sl = 0.0f;
    BalancedState<NG> st;
    softmax_init(st);
    const int t_end = min(len, (t + n) * kTile);
    for (int t0 = t * kTile; t0 < t_end; t0 += piece) {
      const bool head = t0 == t * kTile;
      ring_attend<NG, W, P, kHeadRing, GEN>(a, st, qop, sl, b, h, t0, min(t_end, t0 + piece), len, lane, wave, phase,
                                            lds, [&] {
        if (head) sl = load_head<NG, !kPvMfma && (NG <= 4)>(a, q_dtype, b, h, lane, qop);
      });
    }
    if constexpr (P > 1) __syncthreads();  // every wave is done with the ring: it becomes the merge buffer
    write_partial_heads<NG, HG, P>(a, st, (int64_t(b) + j) * Hkv + h, lane, wave,
                                   reinterpret_cast<float(*)[NG][kHead]>(&lds.ring[0][0][0][0]), s_m, s_l);
    u += n;
    t += n;
    if (t == tb) {
      t = -a.seq_units;
      do ++b; while (b < num_seqs && s_len[b] <= 0);
    }
  }
}

// Max and sum over the 64 lanes of a wave, in every lane: four DPP steps
// inside each 16-lane row, then two swaps across rows.
__device__ __forceinline__ float wave_max(float v) {
  v = __builtin_fmaxf(v, dpp<kDppXor1>(v));
  v = __builtin_fmaxf(v, dpp<kDppXor2>(v));
  v = __builtin_fmaxf(v, dpp<kDppHalfMirror>(v));
  v = __builtin_fmaxf(v, dpp<kDppRowMirror>(v));
  v = __builtin_fmaxf(v, __shfl_xor(v, 16));
  return __builtin_fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// Per sequence, one workgroup per ROWS output rows (row h G + g: query token
// g / heads of the sequence, query head h heads + g % heads), with S waves
// (S = blockDim / 64, chosen by the host from the records a sequence is
// expected to have): wave s takes the s-th of S equal stretches of the
// records.  In a wave, 64 / ROWS lanes serve one output row, lane c of them
// 2 ROWS consecutive columns.  ROWS = 4 (a few records per sequence, batched
// decode) merges four rows per wave, and the combine's time follows its
// number of waves; ROWS = 1 (many records: a long sequence spread over many
// runs) gives each row its own workgroup, so that its records spread over
// more CUs.  The records are taken 64 / ROWS at a time: lane c of the row
// holds record c's maximum and sum, reductions over the row's lanes (with an
// online rescale across chunks) give the weights, and a permute hands each
// weight to the row's lanes; the column loads of a batch of records go out
// together.  With S > 1 the S partial states merge through LDS and wave 0
// writes the output.
constexpr int kCombineMaxWaves = 16;
// Records per round of column loads, per lane: 2 ROWS floats each.
template <int ROWS> constexpr int combine_batch() { return ROWS == 1 ? 16 : 8; }
// Dynamic LDS of a combine workgroup of S waves (nothing for one wave).
template <int ROWS>
constexpr size_t combine_lds_bytes(int64_t S) {
  return S > 1 ? size_t(S) * (2 * ROWS + 64 * 2 * ROWS) * sizeof(float) : 0;
}

// max and sum over the L lanes of each row group of a wave (L = 16 or 64)
template <int L>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (L == 64) return wave_max(v);
  v = __builtin_fmaxf(v, dpp<kDppXor1>(v));
  v = __builtin_fmaxf(v, dpp<kDppXor2>(v));
  v = __builtin_fmaxf(v, dpp<kDppHalfMirror>(v));
  return __builtin_fmaxf(v, dpp<kDppRowMirror>(v));
}
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L == 64) return wave_sum(v);
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v + dpp<kDppRowMirror>(v);
}

template <int OUT_DT, int ROWS>
__global__ void __launch_bounds__(64 * kCombineMaxWaves) decode_combine_kernel(DecodeArgs a) {
  constexpr int L = 64 / ROWS;    // lanes per output row, and records per chunk
  constexpr int CPL = 2 * ROWS;   // columns per lane
  constexpr int NB = combine_batch<ROWS>();
  const int G = a.group;
  const int lane = threadIdx.x & 63;
  const int rr = lane / L, c = lane % L;
  const int fr = int(blockIdx.x) * ROWS + rr;  // this lane's output row
  const bool row_ok = fr < a.num_kv_heads * G;
  const int h = row_ok ? fr / G : 0, g = row_ok ? fr - h * G : 0, b = blockIdx.y;
  const int qi = g / a.heads, gh = g - qi * a.heads;
  // a row past the last, or a query token slot b does not use, merges nothing
  // and writes nothing
  const bool live = row_ok && qi < q_count(a, b);
  const int64_t tok = q_first(a, b) + qi;
  const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int S = int(blockDim.x) / 64;
  const int rec = G * (kHead + 2);
  int64_t first = 0;  // index of the first record of (b, h)
  int64_t rs = rec;   // floats between consecutive records of (b, h)
  int n = 0;          // records of (b, h): the same for every kv head of b
  if (a.stream_wgs > 0) {
    // run j of head h took units [T j / M, T (j+1) / M); unit u belongs to run
    // j(u) = ((u + 1) M - 1) / T, and b owns units [p0, p0 + units), of which
    // the first seq_units carry no work: the runs of its tiles wrote records
    const int64_t p0 = a.prefix[b], units = a.prefix[b + 1] - p0;
    if (units > 0) {
      const int64_t T = a.prefix[gridDim.y];
      const int64_t M = min<int64_t>(a.stream_wgs, T);  // as the partial kernel caps it
      const int64_t u0 = p0 + a.seq_units, u1 = p0 + units - 1;  // first and last tile units
      const int64_t j0 = ((u0 + 1) * M - 1) / T, j1 = ((u1 + 1) * M - 1) / T;
      first = (int64_t(b) + j0) * a.num_kv_heads + h;
      rs = int64_t(a.num_kv_heads) * rec;
      n = int(j1 - j0 + 1);
    }
  } else {
    const int len = a.seq_lens[b];
    n = len > 0 ? min(a.max_splits, (len + a.split - 1) / a.split) : 0;
    first = (int64_t(b) * a.num_kv_heads + h) * a.max_splits;
  }
  const float vd = descale(a.vd, a.vd_b, a.vd_h, b, h);
  const float* part = a.part + first * rec;
  const float* col = part + 2 * G + g * kHead + CPL * c;
  float mx = kNegBig, den = 0.0f;
  float o[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) o[k] = 0.0f;
  const int r_end = int(int64_t(n) * (w + 1) / S);
  for (int c0 = int(int64_t(n) * w / S); c0 < r_end; c0 += L) {  // uniform over the wave
    const int cnt = min(L, r_end - c0);
    float m = kNegBig, l = 0.0f;
    if (live && c < cnt) {
      m = part[int64_t(c0 + c) * rs + g];
      l = part[int64_t(c0 + c) * rs + G + g];
    }
    const float cm = __builtin_fmaxf(mx, group_max<L>(m));
    const float sc = __builtin_amdgcn_exp2f(mx - cm);
    den *= sc;
#pragma unroll
    for (int k = 0; k < CPL; ++k) o[k] *= sc;
    mx = cm;
    const float wl = __builtin_amdgcn_exp2f(m - cm);  // 0 past cnt and on dead rows
    den += group_sum<L>(l * wl);
    for (int s0 = 0; s0 < cnt; s0 += NB) {
      // 8-byte loads: records are G (kHead + 2) floats apart and their columns
      // start 2 G floats in, so only 8-byte alignment holds for every G
      f32x2 x[NB][CPL / 2];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        // past cnt (or on a dead row) re-read a loaded record; its weight is 0
        const int r = live ? c0 + min(s0 + i, cnt - 1) : 0;
        const f32x2* src = reinterpret_cast<const f32x2*>(live ? col + int64_t(r) * rs : a.part);
#pragma unroll
        for (int k = 0; k < CPL / 2; ++k) x[i][k] = src[k];
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        // record s0 + i's weight from lane s0 + i of the row (uniform: readlane)
        const float wi = L == 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), min(s0 + i, L - 1)))
                                 : __shfl(wl, (lane & ~(L - 1)) + min(s0 + i, L - 1));
        const float wk = s0 + i < cnt ? wi : 0.0f;
#pragma unroll
        for (int k = 0; k < CPL / 2; ++k) {
          o[2 * k] = __builtin_fmaf(x[i][k].x, wk, o[2 * k]);
          o[2 * k + 1] = __builtin_fmaf(x[i][k].y, wk, o[2 * k + 1]);
        }
      }
    }
  }
  if (S > 1) {
    // merge the S stretches (a stretch without records holds mx = kNegBig and
    // zero sums, which weigh nothing) through the launch's dynamic LDS
    // (combine_lds_bytes): S x ROWS maxima and sums, then S x 64 lanes x CPL
    // columns; a one-wave workgroup takes none, so many fit on a CU
    extern __shared__ float s_dyn[];
    float* s_mx = s_dyn;
    float* s_den = s_mx + ROWS * S;
    float* s_o = s_den + ROWS * S;
    if (c == 0) {
      s_mx[w * ROWS + rr] = mx;
      s_den[w * ROWS + rr] = den;
    }
#pragma unroll
    for (int k = 0; k < CPL; ++k) s_o[(w * 64 + lane) * CPL + k] = o[k];
    __syncthreads();
    if (w != 0) return;
    float m_all = mx;
    for (int t = 1; t < S; ++t) m_all = __builtin_fmaxf(m_all, s_mx[t * ROWS + rr]);
    den = 0.0f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) o[k] = 0.0f;
    for (int t = 0; t < S; ++t) {
      const float sc = __builtin_amdgcn_exp2f(s_mx[t * ROWS + rr] - m_all);
      den += s_den[t * ROWS + rr] * sc;
#pragma unroll
      for (int k = 0; k < CPL; ++k) o[k] += s_o[(t * 64 + lane) * CPL + k] * sc;
    }
    mx = m_all;
  }
  if (!live) return;
  // no records (an empty sequence): zeros and lse = -inf
  const float inv = den > 0.0f ? vd / den : 0.0f;
  using Bits = typename Elt<OUT_DT>::Bits;
  Bits* dst = reinterpret_cast<Bits*>(a.out + tok * a.out_tok_stride + int64_t(h * a.heads + gh) * a.out_head_stride) +
              CPL * c;
#pragma unroll
  for (int k = 0; k < CPL; ++k) dst[k] = Elt<OUT_DT>::from_f32(o[k] * inv);
  // natural-log sum of exp(s): 2^mx * den in the exp2 domain
  if (c == 0 && a.lse)
    a.lse[int64_t(h * a.heads + gh) * a.lse_head_stride + tok] =
        den > 0.0f ? (mx + __builtin_log2f(den)) * 0.6931471805599453f : -__builtin_inff();
}

// ---- Prefill: many query tokens per sequence ----
//
// psk_paged_prefill_attention computes what the decode reader computes, for
// sequences with more query rows per kv head than one 16-row MFMA tile holds
// (prefill, chunked prefill, long speculative drafts, groups of more than 16
// query heads).  One workgroup per (query block, kv head): kPfWaves waves of
// kPfSets sets of 16 MFMA rows, kPfRows rows in all; row r is query token
// i0 + r / G, query head g = r % G of the block's tq = kPfRows / G tokens, so
// every K/V row of the block's keys is read from the cache once per tq query
// tokens.  The keys stream through two LDS stages of kPfKeys keys, filled by
// the first wave of each SIMD (two 16-byte chunks of K and two of V per
// thread, converted once, exactly, K to bf16 and V to fp16) and consumed by
// every wave, as 256-byte rows:
//   * K: 16-byte chunk c of key t at chunk c ^ (t & 15), so the lanes of one
//     ds_read_b128 phase (consecutive keys, one chunk) hit distinct banks;
//   * V: chunk c of key t at c ^ (2 (t & 7)), read transposed by
//     ds_read_b64_tr_b16 (four keys of one column per lane and read).
// Per 32 keys and 16 rows: S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (two
// 16-key tiles, four MFMAs each, exactly converted FP8 operands as in the
// decode reader), the softmax in the exp2 domain, then O^T = V^T P^T on
// v_mfma_f32_16x16x32_f16 with P rounded to fp16 once (11 significant bits,
// where the decode reader keeps ~16 in a bf16 hi + lo pair and runs P V
// twice; FA3's FP8 path keeps 4).  Transposed products leave each
// lane one query row (lane % 16): its scores, maximum and sum, and output
// columns 16 b + 4 (lane / 16) + r.  The 32-key MFMA step takes as its
// k = 8 s + j (s = lane / 16) key 4 s + j of the first 16-key tile for j < 4
// and key 4 s + j - 4 of the second for j >= 4: the lane's S^T results of the
// two tiles are then its P^T operand as they stand, and one transposed V read
// per tile gives the matching V^T operand.  A row's maximum is fixed by its
// first 32 keys (see the kernel), so the loop has no rescale.
constexpr int kPfWaves = 8;
constexpr int kPfSets = 2;
constexpr int kPfRows = kPfWaves * kPfSets * 16;
constexpr int kPfKeys = 64;  // keys per LDS stage
constexpr int kPfThreads = kPfWaves * 64;
// The first wave of each SIMD loads, converts and stores the stages.  Waves
// w and w + kPfWaves / 2 share a SIMD; the older one issues first and ends
// its blocks of a stage about a quarter of a stage early, so giving it all
// the staging work evens the two out at the barrier.
constexpr int kPfLoaders = kPfThreads / 2;
constexpr int kPfLoads = kPfKeys * 8 / kPfLoaders;  // 16-byte chunks of K (and of V) per loader per stage
static_assert(kPfKeys % 32 == 0 && kPfLoads >= 1 && kPfLoads * kPfLoaders == kPfKeys * 8,
              "a stage is whole 32-key blocks, its chunks spread evenly over the loaders");

constexpr int kPfSortMax = 1024;  // sequences the pre-pass orders by length (more: batch order)

struct PrefillArgs {
  DecodeArgs a;
  const int32_t* blocks;  // [num_seqs + 1]: query blocks before launch position k; the total last
  const int32_t* order;   // [num_seqs]: the sequence at launch position k
  int32_t num_seqs;
  int32_t tq;             // query tokens per block
  int32_t narrow;         // K/V page and row strides below 2^32: offsets from 32 x 32-bit products
};

// The launch order of the query blocks, in one workgroup of 1024 threads:
// sequences by decreasing length (the keys their last block reads; without
// query tokens last), ties in batch order, then each sequence's blocks from
// its last (the most keys, when causal) to its first.  Writes order[k] and
// the exclusive prefix blocks[k] of ceil(n_b / tq) over launch positions,
// blocks[num_seqs] = the total.  Past kPfSortMax sequences the batch order is
// kept.
__global__ void __launch_bounds__(1024) prefill_blocks_kernel(DecodeArgs a, int num_seqs, int tq, int32_t* blocks,
                                                              int32_t* order) {
  __shared__ int32_t s_key[kPfSortMax];
  __shared__ int32_t s_order[kPfSortMax];
  __shared__ int32_t s_wave[16];
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6;
  const bool sorted = num_seqs <= kPfSortMax;
  if (sorted) {
    int key = -1;
    if (tid < num_seqs) key = q_count(a, tid) > 0 ? max(a.seq_lens[tid], 0) : -1;
    s_key[tid] = key;
    __syncthreads();
    if (tid < num_seqs) {
      int rank = 0;
      for (int j = 0; j < num_seqs; ++j) {
        const int kj = s_key[j];
        rank += (kj > key || (kj == key && j < tid)) ? 1 : 0;
      }
      s_order[rank] = tid;
    }
    __syncthreads();
  }
  int carry = 0;
  for (int c0 = 0; c0 < num_seqs; c0 += 1024) {
    const int k = c0 + tid;
    const int b = k < num_seqs ? (sorted ? s_order[k] : k) : 0;
    const int nb = k < num_seqs ? (q_count(a, b) + tq - 1) / tq : 0;
    int x = nb;  // inclusive prefix over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < 16; ++w) {
      const int t = s_wave[w];
      before += w < wave ? t : 0;
      total += t;
    }
    if (k < num_seqs) {
      blocks[k] = carry + before + x - nb;
      order[k] = b;
    }
    carry += total;
    __syncthreads();
  }
  if (tid == 0) blocks[num_seqs] = carry;
}

// The launch position of query block u (blocks[0] = 0 <= u < blocks[num_seqs]):
// the last k with blocks[k] <= u, by a 64-way search of the wave (one round up
// to 64 sequences, two up to 4096).
__device__ __forceinline__ int block_sequence(const int32_t* blocks, int num_seqs, int u, int lane) {
  int lo = 0, n = num_seqs;  // the answer lies in [lo, lo + n) and blocks[lo] <= u
  while (n > 1) {
    const int step = (n + 63) / 64;
    const bool le = lane * step < n && blocks[lo + lane * step] <= u;  // true on a prefix of the lanes
    const uint64_t m = __ballot(le);
    const int last = 63 - __builtin_clzll(m);
    lo += last * step;
    n = min(step, n - last * step);
  }
  return lo;
}

// Byte offsets, from a 16-key V tile of a stage, of this lane's four
// transposed reads (pv_offsets without the ring slot's K half).
__device__ __forceinline__ void pf_v_offsets(int lane, uint32_t (&off)[4]) {
  const int r = lane & 15, s = lane >> 4;
  const int tok = 4 * s + ((r >> 1) & 3);
  const uint32_t row = uint32_t(1024 * (tok >> 3) + 128 * (tok & 7) + 8 * (r & 1));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = 2 * k + (r >= 8 ? 1 : 0);
    off[k] = row + uint32_t(16 * (c ^ (tok & 7)));
  }
}

template <int OUT_DT>
__device__ __forceinline__ void store_row4(char* dst, f32x4 v);
template <>
__device__ __forceinline__ void store_row4<PSK_DTYPE_F32>(char* dst, f32x4 v) {
  *reinterpret_cast<f32x4*>(dst) = v;
}
template <>
__device__ __forceinline__ void store_row4<PSK_DTYPE_BF16>(char* dst, f32x4 v) {
  using E = Elt<PSK_DTYPE_BF16>;
  const uint32_t lo = uint32_t(E::from_f32(v[0])) | (uint32_t(E::from_f32(v[1])) << 16);
  const uint32_t hi = uint32_t(E::from_f32(v[2])) | (uint32_t(E::from_f32(v[3])) << 16);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(dst) = u32x2{lo, hi};
}

template <int Q_DT, int OUT_DT>
__global__ void __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2)))
prefill_attention_kernel(PrefillArgs p) {
  const DecodeArgs& a = p.a;
  __shared__ u32x4 s_k[2][kPfKeys * 16];  // bf16 K rows, chunk c of key t at c ^ (t & 15)
  __shared__ u32x4 s_v[2][kPfKeys * 16];  // fp16 V rows, chunk c of key t at c ^ (2 (t & 7))
  const int lane = int(threadIdx.x) & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int Hkv = a.num_kv_heads;
  const int total = p.blocks[p.num_seqs];
  const int idx = int(blockIdx.x) / Hkv, h = int(blockIdx.x) - idx * Hkv;
  if (idx >= total) return;
  const int k = __builtin_amdgcn_readfirstlane(block_sequence(p.blocks, p.num_seqs, idx, lane));
  const int b = p.order[k];
  // a sequence's blocks from its last (the most keys, when causal) to its first
  const int i0 = (p.blocks[k + 1] - 1 - idx) * p.tq;
  const int n = q_count(a, b);
  const int ni = min(p.tq, n - i0);
  const int64_t qf = q_first(a, b);
  const int L = max(a.seq_lens[b], 0);
  const int G = a.heads;
  // causal: query token i sees keys below base + i (FA's bottom-right alignment)
  const int base = a.causal ? L - n + 1 : L;
  const int key_end = a.causal ? min(max(base + i0 + ni - 1, 0), L) : L;  // keys any row of the block sees
  const int mask_from = a.causal ? min(max(base + i0, 0), L) : L;         // keys every row sees
  const float qd = descale(a.qd, a.qd_b, a.qd_h, b, h);
  const float kd = descale(a.kd, a.kd_b, a.kd_h, b, h);
  const float vd = descale(a.vd, a.vd_b, a.vd_h, b, h);
  // exp2-domain score scale; a negative one is applied as -q~ (exact) times |sl|
  const float sl_signed = a.scale_log2 * qd * kd;
  const float sl = __builtin_fabsf(sl_signed);

  int row_lim[kPfSets];
  bf16x8 qop[kPfSets][4];
#pragma unroll
  for (int s = 0; s < kPfSets; ++s) {
    const int r = (wave * kPfSets + s) * 16 + (lane & 15);
    const int ti = r / G, g = r - ti * G;
    const bool live = ti < ni;
    row_lim[s] = live ? (a.causal ? min(max(base + i0 + ti, 0), L) : L) : 0;
    uint32_t qw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qw[i] = 0;
    if (live)
      load_query_as<Q_DT>(a.q + (qf + i0 + ti) * a.q_tok_stride + int64_t(h * G + g) * a.q_head_stride, qd,
                          32 * (lane >> 4), qw);
    if (sl_signed < 0.0f) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qw[i] ^= 0x80808080u;  // -q~: E4M3 sign bits
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) qop[s][c] = e4m3x8_to_bf16(qw[2 * c], qw[2 * c + 1]);
  }
  // Softmax state per row set.  m is fixed by the row's first 32 keys and
  // never raised, so the hot loop has no rescale and checks nothing: while
  // every lane's share of a row's sum stays below 2^kPfHeadroom, every p
  // (each below that too) is a finite fp16 value (at most 65504) and every
  // sum and accumulator is finite.  A score
  // far above the first keys' maximum makes a share reach it (or overflow),
  // and the workgroup then redoes the row with exact maxima: a pass for the
  // maxima, then the accumulation again.  Rows without a query token keep
  // m = +kBig (every p is 0).
  constexpr float kPfHeadroom = 15.0f;
  constexpr float kBig = 1.0e30f;
  float m[kPfSets], l[kPfSets];
  f32x4 o[kPfSets][8];
  bool live_row[kPfSets];
#pragma unroll
  for (int s = 0; s < kPfSets; ++s) live_row[s] = ((wave * kPfSets + s) * 16 + (lane & 15)) / G < ni;
  auto reset = [&](float m0) {
#pragma unroll
    for (int s = 0; s < kPfSets; ++s) {
      m[s] = live_row[s] ? m0 : kBig;
      l[s] = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) o[s][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };

  // loads, by the loader waves (threads below kPfLoaders): chunk i =
  // threadIdx.x + u * kPfLoaders of a stage (u < kPfLoads) is 16-byte chunk
  // i & 7 of key i >> 3, of K and of V; keys past key_end and rows on
  // missing pages load as zeros
  const int lc = int(threadIdx.x) & 7;
  auto lkey = [&](int u) { return (int(threadIdx.x) + u * kPfLoaders) >> 3; };
  const bool loader = wave < kPfLoaders / 64;
  const int32_t* bt_row = a.block_table + int64_t(b) * a.bt_stride;
  // the table entry as stored (range-checked where it is used, a stage
  // later: a check here would wait for the load, and with it for the K/V
  // loads issued before it)
  auto page_id = [&](int t, int u) -> int32_t {
    const int key = t * kPfKeys + lkey(u);
    if (key >= key_end) return -1;
    const int pi = page_index(a, key);
    return pi < a.bt_width ? bt_row[pi] : -1;
  };
  const uint8_t* kbase = a.k + int64_t(h) * a.k_head + 16 * lc;
  const uint8_t* vbase = a.v + int64_t(h) * a.v_head + 16 * lc;
  auto fetch = [&](int t, int u, int32_t pid, u32x4& kr, u32x4& vr) {
    kr = u32x4(0);
    vr = u32x4(0);
    if (pid >= 0 && pid < a.num_blocks) {
      const int key = t * kPfKeys + lkey(u);
      const int row = a.bs_shift >= 0 ? key & (a.block_size - 1) : key - page_index(a, key) * a.block_size;
      uint64_t ko, vo;
      if (p.narrow) {  // two v_mad_u64_u32 each
        ko = uint64_t(uint32_t(pid)) * uint32_t(a.k_blk) + uint64_t(uint32_t(row)) * uint32_t(a.k_row);
        vo = uint64_t(uint32_t(pid)) * uint32_t(a.v_blk) + uint64_t(uint32_t(row)) * uint32_t(a.v_row);
      } else {
        ko = uint64_t(int64_t(pid) * a.k_blk + int64_t(row) * a.k_row);
        vo = uint64_t(int64_t(pid) * a.v_blk + int64_t(row) * a.v_row);
      }
      kr = *reinterpret_cast<const u32x4*>(kbase + ko);
      vr = *reinterpret_cast<const u32x4*>(vbase + vo);
    }
  };
  // K as bf16 and V as fp16 (both exact), converted once here for every wave
  auto stage_store = [&](int st, int u, const u32x4& kr, const u32x4& vr) {
    const int lk = lkey(u);
    const int ks = lk & 15, vs = 2 * (lk & 7);
    s_k[st][lk * 16 + ((2 * lc) ^ ks)] = __builtin_bit_cast(u32x4, e4m3x8_to_bf16(kr[0], kr[1]));
    s_k[st][lk * 16 + ((2 * lc + 1) ^ ks)] = __builtin_bit_cast(u32x4, e4m3x8_to_bf16(kr[2], kr[3]));
    s_v[st][lk * 16 + ((2 * lc) ^ vs)] = __builtin_bit_cast(u32x4, e4m3x8_to_f16(vr[0], vr[1]));
    s_v[st][lk * 16 + ((2 * lc + 1) ^ vs)] = __builtin_bit_cast(u32x4, e4m3x8_to_f16(vr[2], vr[3]));
  };

  // read side.  K (the A operand of S^T): key kx = lane % 16 of a 16-key
  // tile, chunk 4 (lane / 16) + c for MFMA c.  V^T (the A operand of O^T):
  // ds_read_b64_tr_b16 gives lane i of a 16-lane group element j of the row
  // that lane 4 j + i / 4 of the group addressed, at its element i % 4; lane
  // r of group s addresses key 4 s + r / 4 of the tile, columns 16 c + 4 (r %
  // 4) .. + 3 (chunk 2 c + (r % 4) / 2, half r % 2), so lane i receives column
  // 16 c + i of keys 4 s .. 4 s + 3.
  const int kx = lane & 15, kc0 = 4 * (lane >> 4);
  const int vkey = 4 * (lane >> 4) + (kx >> 2);  // this lane's V row in a 16-key tile
  const uint32_t vrow = uint32_t(256 * vkey + 8 * (kx & 1));
  const int vq = (kx & 3) >> 1, vsw = 2 * (vkey & 7);  // keys 16 j + vkey: (vkey & 7) is the tile-free swizzle

  // raw scores y = q~ . K of the 32 keys from key0 (-inf where masked), the
  // lane's 8 of each row set
  auto scores = [&](auto masked_tag, int st, int key0, int kb, float (&y)[kPfSets][8]) {
    constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kk = 32 * kb + 16 * j + kx;
      bf16x8 kop[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) kop[c] = __builtin_bit_cast(bf16x8, s_k[st][kk * 16 + ((kc0 + c) ^ kx)]);
#pragma unroll
      for (int s = 0; s < kPfSets; ++s) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[c], qop[s][c], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          y[s][4 * j + r] = !MASKED || key0 + 16 * j + kc0 + r < row_lim[s] ? acc[r] : -__builtin_inff();
      }
    }
  };
  // a lane's largest scaled score of a set (sl >= 0: max(y) * sl); IEEE
  // maximum, so no canonicalizing moves, and a NaN score propagates
  auto lane_max = [&](const float (&y)[8]) {
    return __builtin_elementwise_maximum(
               __builtin_elementwise_maximum(__builtin_elementwise_maximum(y[0], y[1]),
                                             __builtin_elementwise_maximum(y[2], y[3])),
               __builtin_elementwise_maximum(__builtin_elementwise_maximum(y[4], y[5]),
                                             __builtin_elementwise_maximum(y[6], y[7]))) * sl;
  };
  auto row_max = [&](float v) {
    v = __builtin_fmaxf(v, __shfl_xor(v, 16));
    return __builtin_fmaxf(v, __shfl_xor(v, 32));
  };
  // FIRST: the block fixes m (the row's maximum of these keys)
  auto block = [&](auto masked_tag, auto first_tag, int st, int key0, int kb) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool FIRST = decltype(first_tag)::value;
    float y[kPfSets][8];
    scores(masked_tag, st, key0, kb, y);
    const char* vb = reinterpret_cast<const char*>(&s_v[st][0]) + 256 * 32 * kb;
    // set by set: set s + 1's softmax (VALU) is independent of set s's P V
    // (MFMA), so the two overlap; V^T is read again for each set rather than
    // held in registers
#pragma unroll
    for (int s = 0; s < kPfSets; ++s) {
      if constexpr (FIRST) m[s] = live_row[s] ? __builtin_fmaxf(row_max(lane_max(y[s])), kNegBig) : kBig;
      // P rounded to fp16 (RNE, relative error <= 2^-11 from 2^-14 up; every
      // p is below 2^15 in the pass that is kept, see the headroom)
      float pv[8], ps = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = __builtin_fmaf(y[s][i], sl, -m[s]);
        pv[i] = __builtin_amdgcn_exp2f(MASKED && y[s][i] == -__builtin_inff() ? -__builtin_inff() : e);
        ps += pv[i];
      }
      l[s] += ps;
      uint32_t pw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pw[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{pv[2 * i], pv[2 * i + 1]}), f16x2));
      const f16x8 pop = __builtin_bit_cast(f16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t off = vrow + uint32_t(16 * ((2 * c + vq) ^ vsw));
        const s16x4 t0 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vb + off));
        const s16x4 t1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vb + 256 * 16 + off));
        const f16x8 vop = __builtin_bit_cast(f16x8, __builtin_shufflevector(t0, t1, 0, 1, 2, 3, 4, 5, 6, 7));
        o[s][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, o[s][c], 0, 0, 0);
      }
    }
    // Ask the scheduler to alternate one MFMA with up to four VALU
    // instructions over the block's 32 MFMAs, so that each wave's softmax
    // issues under its own matrix work as well as under the other wave's.
    // With P V run twice (P as bf16 hi + lo) this was 2-3 % faster on three
    // boxes; with P in fp16, one MFMA to 2, 3 or 4 VALU and no hint measure
    // within 1.5 % of each other and six VALU 2 % slower.
    constexpr int kBlockMfmas = kPfSets * (8 + 8);  // per set: S^T 2 x 4, then P V 8
#pragma unroll
    for (int i = 0; i < kBlockMfmas; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // up to four VALU
    }
  };
  // the maxima pass of a redo: the lane's largest scaled score per set into m
  auto block_max = [&](auto masked_tag, int st, int key0, int kb) {
    float y[kPfSets][8];
    scores(masked_tag, st, key0, kb, y);
#pragma unroll
    for (int s = 0; s < kPfSets; ++s) m[s] = __builtin_fmaxf(m[s], lane_max(y[s]));
  };

  // The keys of the block stream through two LDS stages: the loads of stage
  // t + 1 fly while stage t is consumed, and the page id of stage t + 2 while
  // those land.  Stage 0, the stages every row sees whole and the rest (the
  // causal band and the end of the keys) each run as straight-line code over
  // their 32-key blocks; every wave takes the same (uniform) path, so the
  // barriers match.
  const int n_tiles = (key_end + kPfKeys - 1) / kPfKeys;
  const int t_open = min(n_tiles, mask_from / kPfKeys);  // stages [0, t_open) need no mask
  using T = std::true_type;
  using F = std::false_type;
  // one stage's 32-key blocks.  MODE 0: the pass with m fixed by the first
  // block (FIRST); 1: the maxima of a redo; 2: the accumulation of a redo (m
  // exact)
  auto run_stage = [&](auto mode, auto masked_tag, auto first_tag, int st, int t) {
    constexpr int MODE = decltype(mode)::value;
#pragma unroll
    for (int kb = 0; kb < kPfKeys / 32; ++kb) {
      const int key0 = t * kPfKeys + 32 * kb;
      if (decltype(masked_tag)::value && key0 >= key_end) break;
      if constexpr (MODE == 1) {
        block_max(masked_tag, st, key0, kb);
      } else if (kb == 0) {
        block(masked_tag, first_tag, st, key0, kb);
      } else {
        block(masked_tag, F{}, st, key0, kb);
      }
    }
  };
  auto stream = [&](auto mode) {
    u32x4 kr[kPfLoads], vr[kPfLoads];
    int32_t pid_next[kPfLoads];
#pragma unroll
    for (int u = 0; u < kPfLoads; ++u) pid_next[u] = -1;
    if (n_tiles > 0 && loader) {
      int32_t pid0[kPfLoads];
#pragma unroll
      for (int u = 0; u < kPfLoads; ++u) {
        pid0[u] = page_id(0, u);
        pid_next[u] = n_tiles > 1 ? page_id(1, u) : -1;
      }
#pragma unroll
      for (int u = 0; u < kPfLoads; ++u) fetch(0, u, pid0[u], kr[u], vr[u]);
#pragma unroll
      for (int u = 0; u < kPfLoads; ++u) stage_store(0, u, kr[u], vr[u]);
    }
    __syncthreads();
    auto stage = [&](int t, auto masked_tag, auto first_tag) {
      const bool more = t + 1 < n_tiles && loader;
      if (more) {
#pragma unroll
        for (int u = 0; u < kPfLoads; ++u) fetch(t + 1, u, pid_next[u], kr[u], vr[u]);
#pragma unroll
        for (int u = 0; u < kPfLoads; ++u) pid_next[u] = t + 2 < n_tiles ? page_id(t + 2, u) : -1;
      }
      run_stage(mode, masked_tag, first_tag, t & 1, t);
      if (more) {
#pragma unroll
        for (int u = 0; u < kPfLoads; ++u) stage_store((t + 1) & 1, u, kr[u], vr[u]);
      }
      __syncthreads();
    };
    constexpr bool kFirst = decltype(mode)::value == 0;
    if (n_tiles > 0) {
      if (t_open > 0) stage(0, F{}, std::integral_constant<bool, kFirst>{});
      else stage(0, T{}, std::integral_constant<bool, kFirst>{});
    }
    int t = 1;
    for (; t < t_open; ++t) stage(t, F{}, F{});
    for (; t < n_tiles; ++t) stage(t, T{}, F{});
  };
  reset(kNegBig);
  stream(std::integral_constant<int, 0>{});
  bool ex = false;  // NaN shares also fail the test
#pragma unroll
  for (int s = 0; s < kPfSets; ++s) ex |= !(l[s] < __builtin_ldexpf(1.0f, int(kPfHeadroom)));
  if (__syncthreads_or(ex ? 1 : 0)) {
    // a score past the headroom: exact maxima, then the accumulation again
    reset(kNegBig);
    stream(std::integral_constant<int, 1>{});
    float mx[kPfSets];
#pragma unroll
    for (int s = 0; s < kPfSets; ++s) mx[s] = live_row[s] ? __builtin_fmaxf(row_max(m[s]), kNegBig) : kBig;
    reset(kNegBig);
#pragma unroll
    for (int s = 0; s < kPfSets; ++s) m[s] = mx[s];
    stream(std::integral_constant<int, 2>{});
  }

#pragma unroll
  for (int s = 0; s < kPfSets; ++s) {
    float lt = l[s];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const int r = (wave * kPfSets + s) * 16 + (lane & 15);
    const int ti = r / G, g = r - ti * G;
    if (ti < ni) {
      const int64_t tok = qf + i0 + ti;
      const float inv = lt > 0.0f ? vd / lt : 0.0f;  // a row that sees no key: zeros and lse = -inf
      char* dst = a.out + tok * a.out_tok_stride + int64_t(h * G + g) * a.out_head_stride;
      constexpr int kEsz = Elt<OUT_DT>::kSize;
#pragma unroll
      for (int c = 0; c < 8; ++c) store_row4<OUT_DT>(dst + (16 * c + kc0) * kEsz, o[s][c] * inv);
      if (lane < 16 && a.lse)
        a.lse[int64_t(h * G + g) * a.lse_head_stride + tok] =
            lt > 0.0f ? (m[s] + __builtin_log2f(lt)) * 0.6931471805599453f : -__builtin_inff();
    }
  }
}

template <int Q_DT>
void launch_prefill_q(const PrefillArgs& p, int out_dtype, dim3 grid, hipStream_t st) {
  if (out_dtype == PSK_DTYPE_BF16)
    hipLaunchKernelGGL((prefill_attention_kernel<Q_DT, PSK_DTYPE_BF16>), grid, dim3(kPfThreads), 0, st, p);
  else
    hipLaunchKernelGGL((prefill_attention_kernel<Q_DT, PSK_DTYPE_F32>), grid, dim3(kPfThreads), 0, st, p);
}

// Tokens per workgroup.  num_splits > 0 asks for that many splits of the
// longest sequence; 0 aims at 20 splits of it (measured best for config 2's
// 128 x 8 sequence-heads, within 1% from 17 to 20 and up to 20% slower from 31
// on), more when there are too few sequence-heads to put ~1536 workgroups on a
// long context.  Rounded up to whole 64-token wave
// strides, at least kMinSplit tokens, and doubled until at most kMaxSplits
// splits cover max_seq_len.
int decode_split(int64_t max_seq_len, int64_t num_splits, int64_t seq_heads) {
  const int64_t stride = kTile * kWaves;
  int64_t target = num_splits;
  if (target <= 0) target = std::min<int64_t>(kMaxSplits, std::max<int64_t>(20, ceil_div(1536, std::max<int64_t>(seq_heads, 1))));
  int64_t split = ceil_div(ceil_div(std::max<int64_t>(max_seq_len, 1), target), stride) * stride;
  if (num_splits <= 0) split = std::max<int64_t>(split, kMinSplit);
  while (ceil_div(max_seq_len, split) > kMaxSplits) split *= 2;
  return int(std::min<int64_t>(split, INT32_MAX / 2));
}

// Workgroups of the balanced schedule on the current device: one per slot that
// can be resident at once (CUs x occupancy of the kernel instantiation).  The
// general-page variants launch the same grid, so that the workspace size does
// not depend on the block size.
template <int NG>
int64_t stream_wgs_for() {
  static std::mutex mu;
  static std::map<int, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_partial_stream_kernel<NG, false>, kWaves * 64, 0) !=
          hipSuccess)
    return 0;
  const int64_t n = int64_t(cus) * std::max(per_cu, 1);
  cache[dev] = n;
  return n;
}

int64_t stream_wgs(int ng) {
  switch (ng) {
    case 1: return stream_wgs_for<1>();
    case 2: return stream_wgs_for<2>();
    case 4: return stream_wgs_for<4>();
    case 8: return stream_wgs_for<8>();
    default:
      if constexpr (kPvMfma) return stream_wgs_for<16>();
      return 0;
  }
}

int group_ng(int64_t G) { return G == 1 ? 1 : G == 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 16; }

// kv heads per workgroup of the head-parallel schedule: the largest of 8, 4,
// 2, 1 that divides Hkv.
int heads_hg(int64_t Hkv) { return Hkv % 8 == 0 ? 8 : Hkv % 4 == 0 ? 4 : Hkv % 2 == 0 ? 2 : 1; }

// Resident workgroups of the head-parallel kernel on the current device.
template <int NG, int HG>
int64_t heads_wgs_for() {
  static std::mutex mu;
  static std::map<int, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_partial_heads_kernel<NG, HG, false>, kHeadWaves * 64,
                                                   0) != hipSuccess)
    return 0;
  const int64_t n = int64_t(cus) * std::max(per_cu, 1);
  cache[dev] = n;
  return n;
}

template <int NG>
int64_t heads_wgs_ng(int hg) {
  switch (hg) {
    case 1: return heads_wgs_for<NG, 1>();
    case 2: return heads_wgs_for<NG, 2>();
    case 4: return heads_wgs_for<NG, 4>();
    default: return heads_wgs_for<NG, 8>();
  }
}

// Runs per head group (workgroups that share one head group's units).
int64_t heads_runs(int ng, int64_t num_kv_heads) {
  const int hg = heads_hg(num_kv_heads);
  int64_t slots = 0;
  switch (ng) {
    case 1: slots = heads_wgs_ng<1>(hg); break;
    case 2: slots = heads_wgs_ng<2>(hg); break;
    case 4: slots = heads_wgs_ng<4>(hg); break;
    case 8: slots = heads_wgs_ng<8>(hg); break;
    default:
      if constexpr (kPvMfma) slots = heads_wgs_ng<16>(hg);
      break;
  }
  return slots > 0 ? std::max<int64_t>(1, slots / (num_kv_heads / hg)) : 0;
}

template <int NG, bool GEN>
void launch_heads_ng(const DecodeArgs& a, int q_dtype, int hg, dim3 grid, hipStream_t st, int ns) {
  const dim3 block(kHeadWaves * 64);
  switch (hg) {
    case 1: hipLaunchKernelGGL((decode_partial_heads_kernel<NG, 1, GEN>), grid, block, 0, st, a, q_dtype, ns); break;
    case 2: hipLaunchKernelGGL((decode_partial_heads_kernel<NG, 2, GEN>), grid, block, 0, st, a, q_dtype, ns); break;
    case 4: hipLaunchKernelGGL((decode_partial_heads_kernel<NG, 4, GEN>), grid, block, 0, st, a, q_dtype, ns); break;
    default: hipLaunchKernelGGL((decode_partial_heads_kernel<NG, 8, GEN>), grid, block, 0, st, a, q_dtype, ns); break;
  }
}

// The partial kernels of one schedule for group slot ng: the balanced
// schedule's head-parallel (heads) or per-head kernel with `runs` > 0, else
// one workgroup per (split, kv head, sequence).
template <bool GEN>
void launch_partials(const DecodeArgs& a, int q_dtype, int ng, int64_t runs, bool heads, int64_t num_kv_heads,
                     dim3 grid, hipStream_t st, int ns) {
  const dim3 block(kWaves * 64);
  if (runs > 0 && heads) {
    const int hg = heads_hg(num_kv_heads);
    const dim3 sgrid{unsigned(runs * (num_kv_heads / hg)), 1u, 1u};
    switch (ng) {
      case 1: launch_heads_ng<1, GEN>(a, q_dtype, hg, sgrid, st, ns); break;
      case 2: launch_heads_ng<2, GEN>(a, q_dtype, hg, sgrid, st, ns); break;
      case 4: launch_heads_ng<4, GEN>(a, q_dtype, hg, sgrid, st, ns); break;
      case 8: launch_heads_ng<8, GEN>(a, q_dtype, hg, sgrid, st, ns); break;
      default:
        if constexpr (kPvMfma) launch_heads_ng<16, GEN>(a, q_dtype, hg, sgrid, st, ns);
        break;
    }
  } else if (runs > 0) {
    const dim3 sgrid{unsigned(runs * num_kv_heads), 1u, 1u};
    switch (ng) {
      case 1: hipLaunchKernelGGL((decode_partial_stream_kernel<1, GEN>), sgrid, block, 0, st, a, q_dtype, ns); break;
      case 2: hipLaunchKernelGGL((decode_partial_stream_kernel<2, GEN>), sgrid, block, 0, st, a, q_dtype, ns); break;
      case 4: hipLaunchKernelGGL((decode_partial_stream_kernel<4, GEN>), sgrid, block, 0, st, a, q_dtype, ns); break;
      case 8: hipLaunchKernelGGL((decode_partial_stream_kernel<8, GEN>), sgrid, block, 0, st, a, q_dtype, ns); break;
      default:
        if constexpr (kPvMfma)
          hipLaunchKernelGGL((decode_partial_stream_kernel<16, GEN>), sgrid, block, 0, st, a, q_dtype, ns);
        break;
    }
  } else {
    switch (ng) {
      case 1: hipLaunchKernelGGL((decode_partial_ring_kernel<1, GEN>), grid, block, 0, st, a, q_dtype); break;
      case 2: hipLaunchKernelGGL((decode_partial_ring_kernel<2, GEN>), grid, block, 0, st, a, q_dtype); break;
      case 4: hipLaunchKernelGGL((decode_partial_ring_kernel<4, GEN>), grid, block, 0, st, a, q_dtype); break;
      case 8: hipLaunchKernelGGL((decode_partial_ring_kernel<8, GEN>), grid, block, 0, st, a, q_dtype); break;
      default:
        if constexpr (kPvMfma) hipLaunchKernelGGL((decode_partial_ring_kernel<16, GEN>), grid, block, 0, st, a, q_dtype);
        break;
    }
  }
}

// Workgroups per kv head of the balanced schedule.
int64_t stream_runs(int ng, int64_t num_kv_heads) {
  const int64_t slots = stream_wgs(ng);
  return slots > 0 ? std::max<int64_t>(1, slots / num_kv_heads) : 0;
}

// The head-parallel schedule from kHeadsMinSeqs sequences up; a single
// sequence takes the per-head schedule, whose 4-wave workgroups put more waves
// on it.  Measured with P V on the matrix cores: from 2 sequences the
// head-parallel schedule is faster (2 x 32768 tokens 32.8 us against 35.1,
// 4 x 16384 32.5 against 34.8, 7 mixed 27.5 against 30.8, 3 skewed 45.5
// against 52.4; 6 x 2048 at group 8 20.9 against 19.3), config 2's 128
// sequences 223 us against 266 before it.
constexpr int64_t kHeadsMinSeqs = 2;

// Units that stand for the fixed cost of starting a sequence in a run (see
// units_of), per schedule.
#ifndef PSK_HEADS_SEQ_UNITS
#define PSK_HEADS_SEQ_UNITS 8
#endif
#ifndef PSK_STREAM_SEQ_UNITS
#define PSK_STREAM_SEQ_UNITS 0
#endif
constexpr int kHeadsSeqUnits = PSK_HEADS_SEQ_UNITS;
constexpr int kStreamSeqUnits = PSK_STREAM_SEQ_UNITS;

// Runs per workgroup family of the balanced schedule for this batch.
int64_t balanced_runs(int ng, int64_t num_seqs, int64_t num_kv_heads) {
  return num_seqs >= kHeadsMinSeqs ? heads_runs(ng, num_kv_heads) : stream_runs(ng, num_kv_heads);
}

}  // namespace

extern "C" {

int64_t psk_paged_decode_workspace_len(int64_t num_seqs, int64_t q_len, int64_t num_q_heads, int64_t num_kv_heads,
                                       int64_t max_seq_len, int64_t num_splits) {
  if (num_seqs < 0 || q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads ||
      max_seq_len < 0 || num_splits < 0)
    return PSK_E_ARG;
  const int64_t G = q_len * (num_q_heads / num_kv_heads);  // MFMA rows per (sequence, kv head)
  const int64_t rec = G * (kHead + 2);
  const int64_t splits =
      std::max<int64_t>(1, ceil_div(max_seq_len, decode_split(max_seq_len, num_splits, num_seqs * num_kv_heads)));
  int64_t need = num_seqs * num_kv_heads * splits * rec;
  if (num_splits == 0 && num_seqs <= kStreamMaxSeqs && G <= kMaxRows) {
    // the balanced schedule: a record per (sequence, kv head) and per workgroup, then the units prefix
    need = std::max(need,
                    (num_seqs + balanced_runs(group_ng(G), num_seqs, num_kv_heads)) * num_kv_heads * rec + num_seqs + 1);
  }
  return need;
}

int psk_paged_decode_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride, int q_dtype,
                               const void* k_cache, const void* v_cache, const int64_t* k_strides,
                               const int64_t* v_strides, const int32_t* block_table, int64_t block_table_stride,
                               int64_t block_table_width, const int32_t* seq_lens, int64_t num_seqs,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_size, int64_t block_size,
                               int64_t num_blocks, int64_t max_seq_len, int64_t num_splits, int64_t q_len,
                               const int32_t* cu_seqlens_q, int causal, float softmax_scale, const float* q_descale,
                               const float* k_descale, const float* v_descale, const int64_t* descale_strides,
                               void* out, int64_t out_tok_stride, int64_t out_head_stride, int out_dtype, float* lse,
                               int64_t lse_head_stride, float* workspace, int64_t workspace_len, void* stream) {
  begin_device_call();
  if (num_seqs < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(PSK_E_ARG, "bad head counts (q %lld, kv %lld)", (long long)num_q_heads, (long long)num_kv_heads);
  const int64_t group = num_q_heads / num_kv_heads;
  if (q_len <= 0) return fail(PSK_E_ARG, "q_len %lld", (long long)q_len);
  const int64_t G = group * q_len;  // MFMA rows per (sequence, kv head)
  if (G > kMaxRows)
    return fail(PSK_E_ARG, "query tokens x query heads per kv head must be at most %d (got %lld x %lld)", kMaxRows,
                (long long)q_len, (long long)group);
  if (!kPvMfma && (G > 8 || q_len > 1))
    return fail(PSK_E_ARG, "this build (P V on the VALU) takes one query token and at most 8 heads per kv head");
  if (head_size != kHead) return fail(PSK_E_ARG, "head_size must be %d (got %lld)", kHead, (long long)head_size);
  if (block_size <= 0 || num_blocks <= 0 || num_blocks > INT32_MAX || block_table_width <= 0 || max_seq_len < 0 ||
      max_seq_len > INT32_MAX)
    return fail(PSK_E_ARG, "bad cache geometry");
  if (q_dtype != PSK_DTYPE_FP8_E4M3FN && q_dtype != PSK_DTYPE_BF16 && q_dtype != PSK_DTYPE_F16 &&
      q_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "query dtype %d", q_dtype);
  if (out_dtype != PSK_DTYPE_BF16 && out_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "output dtype %d (bf16 or f32)", out_dtype);
  if (num_seqs == 0) return PSK_OK;
  if (!q || !k_cache || !v_cache || !k_strides || !v_strides || !block_table || !seq_lens || !out || !workspace)
    return fail(PSK_E_ARG, "NULL pointer");
  if (!std::isfinite(softmax_scale)) return fail(PSK_E_ARG, "softmax_scale is not finite");
  const int qsz = dtype_size(q_dtype);
  // 16-byte vector loads: every K/V base and stride, and the query rows
  const uint64_t kv_align[8] = {uint64_t(uintptr_t(k_cache)), uint64_t(uintptr_t(v_cache)), uint64_t(k_strides[0]),
                                uint64_t(k_strides[1]),       uint64_t(k_strides[2]),       uint64_t(v_strides[0]),
                                uint64_t(v_strides[1]),       uint64_t(v_strides[2])};
  if (common_align(kv_align, 8, 16) < 16) return fail(PSK_E_ARG, "K/V caches need 16-byte aligned bases and strides");
  const uint64_t q_align[3] = {uint64_t(uintptr_t(q)), uint64_t(q_tok_stride * qsz), uint64_t(q_head_stride * qsz)};
  if (common_align(q_align, 3, 16) < 16) return fail(PSK_E_ARG, "query rows need 16-byte alignment");
  if (num_splits < 0) return fail(PSK_E_ARG, "num_splits %lld", (long long)num_splits);
  const int64_t need =
      psk_paged_decode_workspace_len(num_seqs, q_len, num_q_heads, num_kv_heads, max_seq_len, num_splits);
  if (workspace_len < need)
    return fail(PSK_E_WORKSPACE, "workspace of %lld floats, need %lld", (long long)workspace_len, (long long)need);

  DecodeArgs a{};
  a.q = static_cast<const char*>(q);
  a.q_tok_stride = q_tok_stride * qsz;
  a.q_head_stride = q_head_stride * qsz;
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.k_blk = k_strides[0];
  a.k_row = k_strides[1];
  a.k_head = k_strides[2];
  a.v_blk = v_strides[0];
  a.v_row = v_strides[1];
  a.v_head = v_strides[2];
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.seq_lens = seq_lens;
  a.num_blocks = int32_t(num_blocks);
  a.block_size = int32_t(block_size);
  a.bs_shift = log2_exact(block_size);
  a.num_kv_heads = int32_t(num_kv_heads);
  a.group = int32_t(G);
  a.heads = int32_t(group);
  a.q_len = int32_t(q_len);
  a.cu_q = cu_seqlens_q;
  a.causal = causal ? 1 : 0;
  a.split = decode_split(max_seq_len, num_splits, num_seqs * num_kv_heads);
  a.max_splits = int32_t(std::max<int64_t>(1, ceil_div(max_seq_len, a.split)));
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  const int64_t zero[6] = {0, 0, 0, 0, 0, 0};
  const int64_t* ds = descale_strides ? descale_strides : zero;
  a.qd = q_descale;
  a.qd_b = ds[0];
  a.qd_h = ds[1];
  a.kd = k_descale;
  a.kd_b = ds[2];
  a.kd_h = ds[3];
  a.vd = v_descale;
  a.vd_b = ds[4];
  a.vd_h = ds[5];
  a.part = workspace;
  a.out = static_cast<char*>(out);
  const int osz = dtype_size(out_dtype);
  a.out_tok_stride = out_tok_stride * osz;
  a.out_head_stride = out_head_stride * osz;
  a.lse = lse;
  a.lse_head_stride = lse_head_stride;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ng = group_ng(G);
  const dim3 grid{unsigned(a.max_splits), unsigned(num_kv_heads), unsigned(num_seqs)};
  // a 16-token tile stays in one page when the block size is a power of two >=
  // 16 (and its rows are within 32-bit offsets): wave-uniform tile addressing;
  // any other block size takes the general-page variants
  const bool uniform = a.bs_shift >= 4 && 16 * std::max(a.k_row, a.v_row) < (int64_t(1) << 31);
  const bool heads = num_seqs >= kHeadsMinSeqs;
  const int64_t runs = num_splits == 0 && num_seqs <= kStreamMaxSeqs ? balanced_runs(ng, num_seqs, num_kv_heads) : 0;
  if (runs > 0) {
    a.stream_wgs = int32_t(runs);
    a.seq_units = heads ? kHeadsSeqUnits : kStreamSeqUnits;
    a.prefix = reinterpret_cast<int32_t*>(workspace + (num_seqs + runs) * num_kv_heads * G * (kHead + 2));
  }
  if (uniform) launch_partials<false>(a, q_dtype, ng, runs, heads, num_kv_heads, grid, st, int(num_seqs));
  else launch_partials<true>(a, q_dtype, ng, runs, heads, num_kv_heads, grid, st, int(num_seqs));
  const int st1 = check_launch("decode partial kernel launch");
  if (st1 != PSK_OK) return st1;
  // waves per workgroup in the combine: one per combine_batch() records a
  // sequence is expected to have, so that a wave's records take one round of
  // loads (the balanced schedule spreads runs / sequences + 1 on average; the
  // split schedule at most max_splits), at most kCombineMaxWaves.  Four rows
  // per wave when one wave suffices, else one row per workgroup.
  const int64_t recs = runs > 0 ? runs / num_seqs + 1 : a.max_splits;
  const bool quad = recs <= combine_batch<4>();
  const int64_t waves = quad ? 1
                             : std::max<int64_t>(1, std::min<int64_t>(kCombineMaxWaves,
                                                                      ceil_div(recs, combine_batch<1>())));
  const int rows = quad ? 4 : 1;
  const dim3 grid2{unsigned(ceil_div(num_kv_heads * G, rows)), unsigned(num_seqs), 1u};
  const dim3 block2{unsigned(64 * waves), 1u, 1u};
  const size_t lds2 = quad ? combine_lds_bytes<4>(waves) : combine_lds_bytes<1>(waves);
  if (out_dtype == PSK_DTYPE_BF16) {
    if (quad) hipLaunchKernelGGL((decode_combine_kernel<PSK_DTYPE_BF16, 4>), grid2, block2, lds2, st, a);
    else hipLaunchKernelGGL((decode_combine_kernel<PSK_DTYPE_BF16, 1>), grid2, block2, lds2, st, a);
  } else {
    if (quad) hipLaunchKernelGGL((decode_combine_kernel<PSK_DTYPE_F32, 4>), grid2, block2, lds2, st, a);
    else hipLaunchKernelGGL((decode_combine_kernel<PSK_DTYPE_F32, 1>), grid2, block2, lds2, st, a);
  }
  return check_launch("decode_combine_kernel launch");
}


int64_t psk_paged_prefill_workspace_len(int64_t num_seqs) { return num_seqs < 0 ? PSK_E_ARG : 2 * num_seqs + 1; }

int psk_paged_prefill_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride, int q_dtype,
                                const void* k_cache, const void* v_cache, const int64_t* k_strides,
                                const int64_t* v_strides, const int32_t* block_table, int64_t block_table_stride,
                                int64_t block_table_width, const int32_t* seq_lens, int64_t num_seqs,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t head_size, int64_t block_size,
                                int64_t num_blocks, int64_t total_q, int64_t max_seqlen_q,
                                const int32_t* cu_seqlens_q, int causal, float softmax_scale, const float* q_descale,
                                const float* k_descale, const float* v_descale, const int64_t* descale_strides,
                                void* out, int64_t out_tok_stride, int64_t out_head_stride, int out_dtype, float* lse,
                                int64_t lse_head_stride, int32_t* workspace, int64_t workspace_len, void* stream) {
  begin_device_call();
  if (num_seqs < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(PSK_E_ARG, "bad head counts (q %lld, kv %lld)", (long long)num_q_heads, (long long)num_kv_heads);
  const int64_t group = num_q_heads / num_kv_heads;
  if (group > kPfRows)
    return fail(PSK_E_ARG, "at most %d query heads per kv head (got %lld)", kPfRows, (long long)group);
  if (max_seqlen_q <= 0 || max_seqlen_q > INT32_MAX) return fail(PSK_E_ARG, "max_seqlen_q %lld", (long long)max_seqlen_q);
  if (total_q < 0 || total_q > INT32_MAX) return fail(PSK_E_ARG, "total_q %lld", (long long)total_q);
  if (!cu_seqlens_q && total_q != num_seqs * max_seqlen_q)
    return fail(PSK_E_ARG, "without cu_seqlens_q every sequence has max_seqlen_q rows (%lld != %lld x %lld)",
                (long long)total_q, (long long)num_seqs, (long long)max_seqlen_q);
  if (head_size != kHead) return fail(PSK_E_ARG, "head_size must be %d (got %lld)", kHead, (long long)head_size);
  if (block_size <= 0 || block_size > INT32_MAX || num_blocks <= 0 || num_blocks > INT32_MAX ||
      block_table_width <= 0)
    return fail(PSK_E_ARG, "bad cache geometry");
  if (q_dtype != PSK_DTYPE_FP8_E4M3FN && q_dtype != PSK_DTYPE_BF16 && q_dtype != PSK_DTYPE_F16 &&
      q_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "query dtype %d", q_dtype);
  if (out_dtype != PSK_DTYPE_BF16 && out_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "output dtype %d (bf16 or f32)", out_dtype);
  if (num_seqs == 0 || total_q == 0) return PSK_OK;
  if (!q || !k_cache || !v_cache || !k_strides || !v_strides || !block_table || !seq_lens || !out || !workspace)
    return fail(PSK_E_ARG, "NULL pointer");
  if (!std::isfinite(softmax_scale)) return fail(PSK_E_ARG, "softmax_scale is not finite");
  if (workspace_len < 2 * num_seqs + 1)
    return fail(PSK_E_WORKSPACE, "workspace of %lld words, need %lld", (long long)workspace_len,
                (long long)(2 * num_seqs + 1));
  const int qsz = dtype_size(q_dtype), osz = dtype_size(out_dtype);
  const uint64_t kv_align[8] = {uint64_t(uintptr_t(k_cache)), uint64_t(uintptr_t(v_cache)), uint64_t(k_strides[0]),
                                uint64_t(k_strides[1]),       uint64_t(k_strides[2]),       uint64_t(v_strides[0]),
                                uint64_t(v_strides[1]),       uint64_t(v_strides[2])};
  if (common_align(kv_align, 8, 16) < 16) return fail(PSK_E_ARG, "K/V caches need 16-byte aligned bases and strides");
  const uint64_t q_align[3] = {uint64_t(uintptr_t(q)), uint64_t(q_tok_stride * qsz), uint64_t(q_head_stride * qsz)};
  if (common_align(q_align, 3, 16) < 16) return fail(PSK_E_ARG, "query rows need 16-byte alignment");
  const uint64_t o_align[3] = {uint64_t(uintptr_t(out)), uint64_t(out_tok_stride * osz),
                               uint64_t(out_head_stride * osz)};
  if (common_align(o_align, 3, 4 * osz) < 4 * osz)
    return fail(PSK_E_ARG, "output rows need %d-byte alignment", 4 * osz);

  PrefillArgs p{};
  DecodeArgs& a = p.a;
  a.q = static_cast<const char*>(q);
  a.q_tok_stride = q_tok_stride * qsz;
  a.q_head_stride = q_head_stride * qsz;
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.k_blk = k_strides[0];
  a.k_row = k_strides[1];
  a.k_head = k_strides[2];
  a.v_blk = v_strides[0];
  a.v_row = v_strides[1];
  a.v_head = v_strides[2];
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.seq_lens = seq_lens;
  a.num_blocks = int32_t(num_blocks);
  a.block_size = int32_t(block_size);
  a.bs_shift = log2_exact(block_size);
  a.num_kv_heads = int32_t(num_kv_heads);
  a.group = int32_t(group);
  a.heads = int32_t(group);
  a.q_len = int32_t(max_seqlen_q);
  a.cu_q = cu_seqlens_q;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  const int64_t zero[6] = {0, 0, 0, 0, 0, 0};
  const int64_t* ds = descale_strides ? descale_strides : zero;
  a.qd = q_descale;
  a.qd_b = ds[0];
  a.qd_h = ds[1];
  a.kd = k_descale;
  a.kd_b = ds[2];
  a.kd_h = ds[3];
  a.vd = v_descale;
  a.vd_b = ds[4];
  a.vd_h = ds[5];
  a.out = static_cast<char*>(out);
  a.out_tok_stride = out_tok_stride * osz;
  a.out_head_stride = out_head_stride * osz;
  a.lse = lse;
  a.lse_head_stride = lse_head_stride;
  p.blocks = workspace;
  p.order = workspace + num_seqs + 1;
  p.num_seqs = int32_t(num_seqs);
  p.tq = int32_t(kPfRows / group);
  constexpr int64_t k32 = int64_t(1) << 32;
  p.narrow = k_strides[0] >= 0 && k_strides[0] < k32 && k_strides[1] >= 0 && k_strides[1] < k32 &&
             v_strides[0] >= 0 && v_strides[0] < k32 && v_strides[1] >= 0 && v_strides[1] < k32;
  // query blocks: at most ceil(total_q / tq) whole ones plus one partial per sequence
  const int64_t max_blocks = ceil_div(total_q, p.tq) + num_seqs;
  if (num_seqs > (INT32_MAX - 1) / 2 || max_blocks * num_kv_heads > INT32_MAX)
    return fail(PSK_E_ARG, "too many query blocks (%lld x %lld kv heads)", (long long)max_blocks,
                (long long)num_kv_heads);

  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(prefill_blocks_kernel, dim3(1), dim3(1024), 0, st, a, int(num_seqs), int(p.tq), workspace,
                     workspace + num_seqs + 1);
  const int st1 = check_launch("prefill_blocks_kernel launch");
  if (st1 != PSK_OK) return st1;
  const dim3 grid{unsigned(max_blocks * num_kv_heads), 1u, 1u};
  switch (q_dtype) {
    case PSK_DTYPE_FP8_E4M3FN: launch_prefill_q<PSK_DTYPE_FP8_E4M3FN>(p, out_dtype, grid, st); break;
    case PSK_DTYPE_BF16: launch_prefill_q<PSK_DTYPE_BF16>(p, out_dtype, grid, st); break;
    case PSK_DTYPE_F16: launch_prefill_q<PSK_DTYPE_F16>(p, out_dtype, grid, st); break;
    default: launch_prefill_q<PSK_DTYPE_F32>(p, out_dtype, grid, st); break;
  }
  return check_launch("prefill_attention_kernel launch");
}

}  // extern "C"
