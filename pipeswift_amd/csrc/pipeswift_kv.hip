// Paged KV-cache data path for MI355X (gfx950, CDNA4): append (MHA/GQA and MLA),
// FP8 E4M3FN quantization fused into the append, block gather, copy_blocks,
// per-tensor amax/scale and the device<->pinned-host page transport.
//
// Every kernel here is a memory-bound byte mover; none is a contraction, so no
// MFMA.  Design points shared by all of them:
//   * wavefront-granular work: one 64-lane wave owns one (token-chunk, part) or
//     one page-unit, so the slot / block-table lookups are wave-uniform scalar
//     loads and the row pointers live in SGPRs;
//   * 16-byte lanes (global_load/store_dwordx4) whenever every base pointer,
//     stride and row length allows it, falling back to 8/4/2/1 bytes;
//   * all loads of a wave are issued before its stores so each lane keeps
//     several 16 B requests in flight against HBM latency;
//   * nontemporal (streaming) loads and stores for data a kernel touches
//     once: the cache rows written here are not re-read by the same kernel,
//     and leaving them dirty in L2 makes every launch pay a write-back at its
//     end (measured: the decode append drops from 3.05 to 2.58 us per launch,
//     the 16.8 MB chunked append from 5.9 to 4.4 us);
//   * 64-bit address arithmetic throughout (a 65536-block fp8 cache is 2^31 B).
//
// C ABI: include/pipeswift_kv.h.  Nothing here allocates device memory or
// synchronizes a stream.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "pipeswift_kv.h"
#include "psk_common.h"

// Message of the calling thread's most recent failure (psk_last_error).
thread_local char psk_detail::g_err[512] = "";

using namespace psk_detail;

namespace {

// ----------------------------------------------------------------------------
// paged scatter: append (MHA/GQA, two parts K and V) and MLA concat (two parts
// kv_c and k_pe into one row)
// ----------------------------------------------------------------------------

struct ScatterPart {
  const char* src;      // row 0 of this part's input
  char* dst;            // cache base this part writes into
  const float* scale;   // FP8 scale (device) or nullptr for 1.0
  int64_t src_stride;   // bytes between consecutive input token rows
  int64_t blk_stride;   // bytes between cache blocks
  int64_t page_stride;  // bytes between consecutive slots of a block
  int64_t dst_off;      // bytes from the slot's row start to this part
  int64_t seg_stride;   // cache bytes between segments (heads)
  int64_t inner_stride; // cache bytes between consecutive output vectors of a segment
  int32_t nseg;         // segments per row
  int32_t seg_vecs;     // vectors per segment
};

struct ScatterGeom {
  const int64_t* slots;
  int64_t num_tokens;
  int64_t block_size;
  int64_t num_slots;    // num_blocks * block_size
  int32_t bs_shift;     // log2(block_size), or -1 when not a power of two
  int32_t nparts;       // 1 or 2
  int32_t slice_shift;  // log2(waves per (token chunk, part))
};

// One wave per (chunk of CH tokens, part, slice).  A part's row of `total`
// vectors is cut into 2^slice_shift slices of 64*U vectors (a slice loops when
// the row is longer), so decode-sized batches spread one row over several
// waves and prefill-sized ones give each wave CH rows.
template <class C, int CH, int U, bool FAST, int WPB>
__global__ void __launch_bounds__(WPB * 64) paged_scatter_kernel(ScatterGeom g, ScatterPart p0, ScatterPart p1) {
  // No branch before the row loads: a wave with nothing to do runs with its
  // lanes predicated off, so the scalar loads of the argument segment can
  // issue as one batch.  The workgroup size is a compile-time constant (WPB
  // waves), which keeps blockDim out of the argument segment reads.
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = int64_t(blockIdx.x) * WPB + __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
  const int slice = int(wave & ((int64_t(1) << g.slice_shift) - 1));
  const int64_t rest = wave >> g.slice_shift;
  const bool two = g.nparts == 2;
  const int part = two ? int(rest & 1) : 0;
  const int64_t t0 = (two ? (rest >> 1) : rest) * CH;
  const char* src = part ? p1.src : p0.src;
  char* dst = part ? p1.dst : p0.dst;
  const float* scale_p = part ? p1.scale : p0.scale;
  const int64_t src_stride = part ? p1.src_stride : p0.src_stride;
  const int64_t blk_stride = part ? p1.blk_stride : p0.blk_stride;
  const int64_t page_stride = part ? p1.page_stride : p0.page_stride;
  const int64_t dst_off = part ? p1.dst_off : p0.dst_off;
  const int64_t seg_stride = FAST ? 0 : (part ? p1.seg_stride : p0.seg_stride);
  const int64_t inner_stride = FAST ? C::OUT_B : (part ? p1.inner_stride : p0.inner_stride);
  const int nseg = FAST ? 1 : (part ? p1.nseg : p0.nseg);
  const int seg_vecs = part ? p1.seg_vecs : p0.seg_vecs;
  const bool flat = FAST || (nseg == 1 && inner_stride == C::OUT_B);
  const int total = nseg * seg_vecs;
  const int step = (kWave * U) << g.slice_shift;
  int base = slice * (kWave * U);

  // The input rows do not depend on the slots: their loads are issued first
  // so the slot lookups (scalar loads) overlap the HBM latency of the data.
  bool tv[CH];
  const char* srow[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    tv[c] = t0 + c < g.num_tokens;
    srow[c] = src + (t0 + c) * src_stride;
  }
  typename C::In v[CH][U];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * kWave + lane;
      if (tv[c] && i < total) v[c][u] = vload_nt<C::IN_B>(srow[c] + int64_t(i) * C::IN_B);
    }
  }

  char* drow[CH];
  bool ok[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int64_t slot = tv[c] ? g.slots[t0 + c] : int64_t(-1);
    ok[c] = slot >= 0 && slot < g.num_slots;
    int64_t blk, off;
    if (FAST || g.bs_shift >= 0) {
      blk = slot >> g.bs_shift;
      off = slot & (g.block_size - 1);
    } else {
      blk = slot / g.block_size;
      off = slot - blk * g.block_size;
    }
    drow[c] = dst + blk * blk_stride + off * page_stride + dst_off;
  }
  const QScale qs = make_qscale_uniform(scale_p ? *scale_p : 1.0f);

  for (;;) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * kWave + lane;
        if (ok[c] && i < total) {
          int64_t o;
          if (flat) {
            o = int64_t(i) * C::OUT_B;
          } else {
            const int sg = i / seg_vecs;
            o = int64_t(sg) * seg_stride + int64_t(i - sg * seg_vecs) * inner_stride;
          }
          vstore_nt<C::OUT_B>(drow[c] + o, C::apply(v[c][u], qs));
        }
      }
    }
    base += step;
    if (base >= total) break;
    // rows longer than one pass of the slice: next stretch
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * kWave + lane;
        if (tv[c] && i < total) v[c][u] = vload_nt<C::IN_B>(srow[c] + int64_t(i) * C::IN_B);
      }
    }
  }
}

// Launch shape.  Decode-sized batches (< 1024 tokens) are latency bound: one
// vector per lane (U = 1) and rows split over as many slices as they have
// 64-vector stretches, so e.g. 128 tokens x (K, V) x 1024 bf16 -> 512 waves.
// Larger batches give each wave 4 tokens and 2 vectors per lane (2 tokens and
// one vector when the append quantizes, see launch_scatter).
struct ScatterShape {
  int ch;
  int u;
  int slice_shift;
};

ScatterShape scatter_shape(int64_t num_tokens, int total_vecs) {
  ScatterShape sh;
  if (num_tokens < 1024) {
    sh.ch = 1;
    sh.u = 1;
    int slices = int(ceil_div(total_vecs, kWave));
    if (slices > 8) slices = 8;
    sh.slice_shift = 0;
    while ((1 << sh.slice_shift) < slices) ++sh.slice_shift;
  } else {
    sh.ch = 4;
    sh.u = 2;
    sh.slice_shift = 0;
  }
  return sh;
}

int64_t lds_per_cu();

template <class C, int CH, int U, bool FAST, int WPB>
int launch_scatter_shape(ScatterGeom g, const ScatterPart& p0, const ScatterPart& p1, int slice_shift,
                         hipStream_t st) {
  g.slice_shift = slice_shift;
  const int64_t waves = (ceil_div(g.num_tokens, CH) * g.nparts) << slice_shift;
  const int64_t grid = ceil_div(waves, WPB);
  // Prefill-sized copies (no quantizer) run best at two resident workgroups
  // per CU, set through dynamic LDS: 32768 tokens of config 2's geometry 48.7
  // against 50.4 us uncapped, 131072 tokens 185.5 against 196.3 (5.80 TB/s);
  // one per CU is slower, and the quantizing append needs every wave it can
  // get to cover its VALU work (2 per CU: 70.9 against 39.9 us).
  size_t lds = 0;
  if (C::OUT_B == C::IN_B && g.num_tokens >= 8192) {
    const int64_t l = lds_per_cu();
    if (l > 0) lds = size_t(l / 3 + 1024);
  }
  hipLaunchKernelGGL((paged_scatter_kernel<C, CH, U, FAST, WPB>), dim3(grid), dim3(WPB * kWave), lds, st, g, p0, p1);
  return check_launch("paged_scatter_kernel launch");
}

// Decode-sized appends (< 1024 tokens, power-of-two block size, flat rows of
// at most 512 vectors): the time is latency, so everything the wave needs sits
// in one padding-free argument block that arrives in one round of scalar
// loads (the general kernel's two part structs make the compiler split its
// argument loads into two dependent rounds).  One wave per (token, part,
// slice); the part is the wave number's low bit.  With one wave per workgroup
// every wave of the exact grid is valid, so the row load is issued before any
// argument-dependent branch; with four, the last workgroup's spare waves leave
// first.
struct SmallAppend {
  const int64_t* slots;
  uint64_t num_slots;       // num_blocks * block_size; slot >= num_slots (or < 0) is skipped
  int64_t blk_stride;       // bytes, shared by both parts
  int64_t page_stride;      // bytes, shared by both parts
  const char* src[2];
  char* dst[2];             // cache base + the part's byte offset within a slot row
  const float* scale[2];    // FP8 scale per part, nullptr for 1.0
  int64_t src_stride[2];    // bytes between input token rows
  int32_t vecs[2];          // vectors in each part's row
  int32_t bs_shift;         // log2(block_size)
  int32_t slice_shift;      // log2(slices per row); slices * 64 >= vecs
};

// The amax finish an append can take over from amax_finalize_kernel: the
// partial maxima of K (ws[0, nparts)) and V (ws[stride, stride + nparts)),
// reduced by every wave for its own part, scale = amax / qmax (1.0 for an
// all-zero part) written by the waves of token 0.
struct AmaxFinish {
  const uint32_t* ws;
  int64_t stride;
  int32_t nparts;
  float qmax;
  float* scale_out;  // [2]
  float* amax_out;   // [2] or nullptr
};

// launch_scatter's answer when the fused finish does not apply to the shape:
// nothing was launched, and the caller finalizes the scales and appends.  It
// is no status a call returns: PSK_E_* codes are negative and HIP errors
// (hipError_t values, returned as they are) lie far below 2^20.
constexpr int kNeedScales = 1 << 20;

template <class C, int WPB, bool FIN>
__device__ __forceinline__ void small_append(const SmallAppend& a, const AmaxFinish& f, uint32_t num_waves) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
  if (WPB > 1 && wave >= num_waves) return;  // the last workgroup's spare waves
  const int part = int(wave & 1u);
  const uint32_t rest = wave >> 1;
  const int slice = int(rest & ((1u << a.slice_shift) - 1u));
  const int64_t t = int64_t(rest >> a.slice_shift);
  const int i = slice * kWave + lane;
  // selects, not a[part]: an indexed kernel argument is fetched with vector loads
  const char* src = part ? a.src[1] : a.src[0];
  char* dst = part ? a.dst[1] : a.dst[0];
  const float* sp = part ? a.scale[1] : a.scale[0];
  const int64_t src_stride = part ? a.src_stride[1] : a.src_stride[0];
  const int vecs = part ? a.vecs[1] : a.vecs[0];
  const bool act = i < vecs;
  // every lane loads (lanes past the row re-read its last vector), so no
  // branch delays the row load behind the argument loads
  const int il = act ? i : vecs - 1;
  const typename C::In v = vload_nt<C::IN_B>(src + t * src_stride + int64_t(il) * C::IN_B);
  const int64_t slot = a.slots[t];
  float s;
  if constexpr (FIN) {
    // the part's amax from its partial maxima (abs bit patterns, NaN as 0),
    // as amax_finalize_kernel takes it, while the row is in flight
    const uint32_t* pm = f.ws + (part ? f.stride : 0);
    uint32_t m = 0;
    for (int k = lane; k < f.nparts; k += kWave) {
      const uint32_t q = pm[k];
      m = q > m ? q : m;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const uint32_t o = uint32_t(__shfl_xor(int(m), off, kWave));
      m = o > m ? o : m;
    }
    const float amax = __uint_as_float(uint32_t(__builtin_amdgcn_readfirstlane(int(m))));
    s = amax > 0.0f ? amax / f.qmax : 1.0f;
    if (t == 0 && slice == 0 && lane == 0) {
      f.scale_out[part] = s;
      if (f.amax_out) f.amax_out[part] = amax;
    }
  } else {
    s = sp ? *sp : 1.0f;
  }
  const QScale qs = make_qscale_uniform(s);
  if (act && uint64_t(slot) < a.num_slots) {
    char* drow = dst + (slot >> a.bs_shift) * a.blk_stride +
                 (slot & ((int64_t(1) << a.bs_shift) - 1)) * a.page_stride;
    vstore_nt<C::OUT_B>(drow + int64_t(i) * C::OUT_B, C::apply(v, qs));
  }
}

template <class C, int WPB>
__global__ void __launch_bounds__(64 * WPB) paged_append_small_kernel(SmallAppend a, uint32_t num_waves) {
  small_append<C, WPB, false>(a, AmaxFinish{}, num_waves);
}

// The same append with the scales finished in-kernel from the amax partials:
// one launch fewer than amax_finalize_kernel followed by the append.
template <class C, int WPB>
__global__ void __launch_bounds__(64 * WPB) paged_append_small_amax_kernel(SmallAppend a, AmaxFinish f,
                                                                           uint32_t num_waves) {
  small_append<C, WPB, true>(a, f, num_waves);
}

// Prefill-sized two-part rows whose second part is short (the MLA latent row:
// kv_c 64 vectors + k_pe 8 vectors of 16 input bytes).  One wave per (token
// chunk, part) would leave 7/8 of every k_pe wave's lanes idle while it pays
// the whole wave's instructions, which for the quantizing append is the
// dominant cost.  Here the lanes are packed over the flat (token, vector)
// space of both parts -- vector j of token t is number t * V + j, the first
// V0 from part 0 -- so every lane of every wave moves a vector.  Each lane
// loads its tokens' slots (a lane-varying load; lanes of one token share the
// line), then its U vectors, then stores.  Both parts write one cache (same
// block and slot strides) with one scale, as the MLA entry passes them.
//
// a * b for a, b < 2^24, product taken modulo 2^32 (v_mul_u32_u24: full rate)
__device__ __forceinline__ uint32_t mul24(uint32_t a, uint32_t b) { return uint32_t(__umul24(a, b)); }

template <class C, int V, int V0, int U, bool NARROW>
__global__ void __launch_bounds__(256) packed_row_scatter_kernel(ScatterGeom g, ScatterPart p0, ScatterPart p1) {
  // NARROW: every input part and the cache span less than 4 GiB and every
  // stride, token index and block count fits 24 bits (checked on the host),
  // so offsets are 32-bit and come from full-rate 24-bit multiply-adds instead
  // of the quarter-rate 64-bit products, a third of the kernel's VALU time.
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = blockIdx.x * 4u + uint32_t(__builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave));
  const uint32_t total = uint32_t(g.num_tokens) * uint32_t(V);
  uint32_t tok[U];
  int vec[U];
  const char* src[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t f = wave * uint32_t(kWave * U) + uint32_t(u * kWave + lane);
    const uint32_t fc = f < total ? f : total - 1;  // lanes past the end re-read the last vector
    tok[u] = fc / uint32_t(V);
    const int j = int(fc - tok[u] * uint32_t(V));
    vec[u] = f < total ? j : -1;
    const bool first = j < V0;
    if constexpr (NARROW) {
      const uint32_t stride = uint32_t(first ? p0.src_stride : p1.src_stride);
      src[u] = (first ? p0.src : p1.src) + (mul24(tok[u], stride) + uint32_t(first ? j : j - V0) * C::IN_B);
    } else {
      src[u] = first ? p0.src + int64_t(tok[u]) * p0.src_stride + int64_t(j) * C::IN_B
                     : p1.src + int64_t(tok[u]) * p1.src_stride + int64_t(j - V0) * C::IN_B;
    }
  }
  // The slots load before the rows: loads return in order, so the store
  // offsets are formed while the rows are still in flight.
  int64_t slot[U];
#pragma unroll
  for (int u = 0; u < U; ++u) slot[u] = g.slots[tok[u]];
  typename C::In v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = vload_nt<C::IN_B>(src[u]);
  QScale qs = make_qscale_uniform(p0.scale ? *p0.scale : 1.0f);
  // The empty asm statements keep the reciprocal's division and the store
  // offsets here, under the row loads: left alone, the compiler moves both
  // into the store's branch, behind the wait for the rows.
  asm volatile("" : "+v"(qs.r));
  char* dst[U];
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = vec[u];
    ok[u] = j >= 0 && uint64_t(slot[u]) < uint64_t(g.num_slots);
    if constexpr (NARROW) {
      const uint32_t s32 = uint32_t(slot[u]);
      const uint32_t o = j < V0 ? uint32_t(j) * C::OUT_B : uint32_t(p1.dst_off) + uint32_t(j - V0) * C::OUT_B;
      uint32_t off = mul24(s32 >> g.bs_shift, uint32_t(p0.blk_stride)) +
                     mul24(s32 & uint32_t(g.block_size - 1), uint32_t(p0.page_stride)) + o;
      asm volatile("" : "+v"(off));
      dst[u] = p0.dst + off;
    } else {
      const int64_t sl = slot[u];
      const int64_t o = j < V0 ? int64_t(j) * C::OUT_B : p1.dst_off + int64_t(j - V0) * C::OUT_B;
      dst[u] = p0.dst + (sl >> g.bs_shift) * p0.blk_stride + (sl & (g.block_size - 1)) * p0.page_stride + o;
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (ok[u]) vstore_nt<C::OUT_B>(dst[u], C::apply(v[u], qs));
}

// The packed launch applies to the quantizing append of flat two-part rows of
// 64 + 8 vectors into one cache with power-of-two pages and one scale, from
// 1024 tokens up (decode-sized batches take paged_append_small_kernel).  One
// vector per lane: config 4's FP8 prefill (4096 tokens) 3.20 us against 3.54
// with one wave per (2 tokens, part), and 3.49 / 4.14 at two / four vectors
// per lane.  The bf16 copy of the same rows stays on the per-part waves
// (3.10 us against 3.68 packed), where no per-wave arithmetic is saved.
template <class C>
bool launch_packed_rows(const ScatterGeom& g, const ScatterPart& p0, const ScatterPart& p1, hipStream_t st,
                        int* status) {
  constexpr int U = 1;
  if (C::OUT_B >= C::IN_B || g.nparts != 2 || g.bs_shift < 0 || g.num_tokens < 1024 || p0.seg_vecs != 64 ||
      p1.seg_vecs != 8 || p0.dst != p1.dst || p0.dst_off != 0 || p0.blk_stride != p1.blk_stride ||
      p0.page_stride != p1.page_stride || p0.scale != p1.scale ||
      g.num_tokens > (int64_t(INT32_MAX) - 4 * kWave * U) / 72)
    return false;
  const int64_t waves = ceil_div(g.num_tokens * 72, kWave * U);
  // 32-bit offsets when every span fits (see the kernel)
  constexpr int64_t k24 = int64_t(1) << 24, k32 = int64_t(1) << 32;
  const int64_t num_blocks = g.num_slots >> g.bs_shift;
  const int64_t row_in = int64_t(p0.seg_vecs) * C::IN_B, row_k = int64_t(p1.seg_vecs) * C::IN_B;
  const int64_t cache_span = (num_blocks - 1) * p0.blk_stride + (g.block_size - 1) * p0.page_stride +
                             p1.dst_off + int64_t(p1.seg_vecs) * C::OUT_B;
  const bool narrow = g.num_tokens <= k24 && g.num_slots < (int64_t(1) << 31) && num_blocks < k24 &&
                      g.block_size < k24 && p0.blk_stride >= 0 && p0.blk_stride < k24 && p0.page_stride >= 0 && p0.page_stride < k24 &&
                      p0.src_stride >= 0 && p0.src_stride < k24 && p1.src_stride >= 0 && p1.src_stride < k24 &&
                      (g.num_tokens - 1) * p0.src_stride + row_in < k32 &&
                      (g.num_tokens - 1) * p1.src_stride + row_k < k32 && cache_span < k32 && p1.dst_off < k24;
  if (narrow)
    hipLaunchKernelGGL((packed_row_scatter_kernel<C, 72, 64, U, true>), dim3(ceil_div(waves, 4)), dim3(4 * kWave), 0,
                       st, g, p0, p1);
  else
    hipLaunchKernelGGL((packed_row_scatter_kernel<C, 72, 64, U, false>), dim3(ceil_div(waves, 4)), dim3(4 * kWave), 0,
                       st, g, p0, p1);
  *status = check_launch("packed_row_scatter_kernel launch");
  return true;
}

bool part_flat(const ScatterPart& p, int out_b) { return p.nseg == 1 && p.inner_stride == out_b; }

// fin: finish the amax scales in the append's own waves (the small kernel
// only; other shapes return kNeedScales having launched nothing).
template <class C>
int launch_scatter(const ScatterGeom& g, const ScatterPart& p0, const ScatterPart& p1, hipStream_t st,
                   const AmaxFinish* fin = nullptr) {
  const int total = p0.nseg * p0.seg_vecs > p1.nseg * p1.seg_vecs ? p0.nseg * p0.seg_vecs : p1.nseg * p1.seg_vecs;
  const ScatterShape sh = scatter_shape(g.num_tokens, total);
  const bool fast = g.bs_shift >= 0 && part_flat(p0, C::OUT_B) && (g.nparts == 1 || part_flat(p1, C::OUT_B));
  const bool small = fast && sh.ch == 1 && g.nparts == 2 && total <= 8 * kWave && p0.blk_stride == p1.blk_stride &&
                     p0.page_stride == p1.page_stride && g.num_tokens <= INT32_MAX / 16;
  if (fin && !(small && C::OUT_B < C::IN_B)) return kNeedScales;
  if (!fast) return launch_scatter_shape<C, 1, 2, false, 4>(g, p0, p1, sh.ch == 1 ? sh.slice_shift : 0, st);
  if (small) {
    SmallAppend a;
    a.slots = g.slots;
    a.num_slots = uint64_t(g.num_slots);
    a.blk_stride = p0.blk_stride;
    a.page_stride = p0.page_stride;
    const ScatterPart* pp[2] = {&p0, &p1};
    for (int k = 0; k < 2; ++k) {
      a.src[k] = pp[k]->src;
      a.dst[k] = pp[k]->dst + pp[k]->dst_off;
      a.scale[k] = pp[k]->scale;
      a.src_stride[k] = pp[k]->src_stride;
      a.vecs[k] = pp[k]->seg_vecs;
    }
    a.bs_shift = g.bs_shift;
    a.slice_shift = sh.slice_shift;
    // One wave per workgroup up to 1024 waves, four from 2048 (measured: config 1's
    // 2048 waves 2.48 us at four against 2.61 at one; config 2's 1024 waves 2.21
    // at one against 2.25 at four).
    const int64_t waves = (g.num_tokens * 2) << sh.slice_shift;
    if (fin) {
      if (waves >= 2048)
        hipLaunchKernelGGL((paged_append_small_amax_kernel<C, 4>), dim3(ceil_div(waves, 4)), dim3(4 * kWave), 0, st,
                           a, *fin, uint32_t(waves));
      else
        hipLaunchKernelGGL((paged_append_small_amax_kernel<C, 1>), dim3(waves), dim3(kWave), 0, st, a, *fin,
                           uint32_t(waves));
      return check_launch("paged_append_small_amax_kernel launch");
    }
    if (waves >= 2048)
      hipLaunchKernelGGL((paged_append_small_kernel<C, 4>), dim3(ceil_div(waves, 4)), dim3(4 * kWave), 0, st, a,
                         uint32_t(waves));
    else
      hipLaunchKernelGGL((paged_append_small_kernel<C, 1>), dim3(waves), dim3(kWave), 0, st, a, uint32_t(waves));
    return check_launch("paged_append_small_kernel launch");
  }
  if (sh.ch == 1) return launch_scatter_shape<C, 1, 1, true, 1>(g, p0, p1, sh.slice_shift, st);
  int packed_status;
  if (launch_packed_rows<C>(g, p0, p1, st, &packed_status)) return packed_status;
  // A quantizing append gets one token per wave and one vector per lane (a row
  // longer than 64 vectors loops): 32768 prefill tokens of config 2's geometry
  // 38.6 us against 39.8 at two tokens per wave, 40.9 at two vectors per lane
  // (a whole row in one pass), and 150.0 against 152.7 us at 131072 tokens.
  // Four tokens and two vectors per lane stay best for the plain copies.
  if constexpr (C::OUT_B < C::IN_B) return launch_scatter_shape<C, 1, 1, true, 4>(g, p0, p1, 0, st);
  return launch_scatter_shape<C, 4, 2, true, 4>(g, p0, p1, sh.slice_shift, st);
}

// Dispatch on (in_dtype, cache_dtype, vector elements).
int dispatch_scatter(int in_dt, int cache_dt, int elems, const ScatterGeom& g, const ScatterPart& p0,
                     const ScatterPart& p1, hipStream_t st, const AmaxFinish* fin = nullptr) {
  if (in_dt == cache_dt) {
    if (fin) return kNeedScales;
    switch (elems * dtype_size(in_dt)) {
      case 16: return launch_scatter<CopyConv<16>>(g, p0, p1, st);
      case 8: return launch_scatter<CopyConv<8>>(g, p0, p1, st);
      case 4: return launch_scatter<CopyConv<4>>(g, p0, p1, st);
      case 2: return launch_scatter<CopyConv<2>>(g, p0, p1, st);
      case 1: return launch_scatter<CopyConv<1>>(g, p0, p1, st);
    }
    return fail(PSK_E_ARG, "internal: bad copy vector width");
  }
  if (cache_dt != PSK_DTYPE_FP8_E4M3FN) return fail(PSK_E_DTYPE, "cache dtype must equal the input dtype or be fp8_e4m3fn");
#define PSK_QUANT_CASES(DT)                                                   \
  switch (elems) {                                                            \
    case 8: return launch_scatter<QuantConv<DT, 8>>(g, p0, p1, st, fin);      \
    case 4: return launch_scatter<QuantConv<DT, 4>>(g, p0, p1, st, fin);      \
    case 2: return launch_scatter<QuantConv<DT, 2>>(g, p0, p1, st, fin);      \
    case 1: return launch_scatter<QuantConv<DT, 1>>(g, p0, p1, st, fin);      \
  }                                                                           \
  return fail(PSK_E_ARG, "internal: bad quant vector width");
  switch (in_dt) {
    case PSK_DTYPE_BF16: { PSK_QUANT_CASES(PSK_DTYPE_BF16) }
    case PSK_DTYPE_F16: { PSK_QUANT_CASES(PSK_DTYPE_F16) }
    case PSK_DTYPE_F32: {
      switch (elems) {
        case 4: return launch_scatter<QuantConv<PSK_DTYPE_F32, 4>>(g, p0, p1, st, fin);
        case 2: return launch_scatter<QuantConv<PSK_DTYPE_F32, 2>>(g, p0, p1, st, fin);
        case 1: return launch_scatter<QuantConv<PSK_DTYPE_F32, 1>>(g, p0, p1, st, fin);
      }
      return fail(PSK_E_ARG, "internal: bad quant vector width");
    }
  }
#undef PSK_QUANT_CASES
  return fail(PSK_E_DTYPE, "fp8 append needs a bf16, fp16 or fp32 input");
}

// Largest vector (in elements) such that every input address/stride is a
// multiple of elems*in_size bytes and every output one of elems*out_size bytes.
int pick_elems(int in_size, int out_size, const std::vector<uint64_t>& in_bytes,
               const std::vector<uint64_t>& out_bytes, int64_t seg_elems) {
  int e = 16 / in_size;
  if (16 / out_size < e) e = 16 / out_size;
  while (e > 1) {
    bool ok = (seg_elems % e) == 0;
    for (uint64_t v : in_bytes) ok = ok && (v % uint64_t(e * in_size)) == 0;
    for (uint64_t v : out_bytes) ok = ok && (v % uint64_t(e * out_size)) == 0;
    if (ok) break;
    e >>= 1;
  }
  return e;
}

// ----------------------------------------------------------------------------
// paged gather: block table -> contiguous rows
// ----------------------------------------------------------------------------

struct GatherGeom {
  const char* src0;
  const char* src1;
  char* dst0;
  char* dst1;
  const int32_t* block_table;
  const int32_t* cu;
  const int32_t* starts;
  const float* scale;
  int64_t batch;
  int64_t bt_stride;
  int64_t num_tokens;
  int64_t block_size;
  int64_t num_blocks;
  int64_t blk_stride;   // bytes
  int64_t page_stride;  // bytes
  int64_t dst_stride;   // bytes
  int32_t row_vecs;
  int32_t bs_shift;
  int32_t nparts;
};

template <class C, int CH, int U, bool POW2>
__global__ void __launch_bounds__(256) paged_gather_kernel(GatherGeom g) {
  const int lane = threadIdx.x & (kWave - 1);
  // Part 0 (K) fills the first half of the grid and part 1 (V) the second, so
  // the waves in flight at any time stream one part's pages into one
  // contiguous output (config 3: 116.5 us against 118.5 with the parts
  // interleaved wave by wave).  The launch gives each part the same number of
  // workgroups.
  const int64_t half = gridDim.x >> 1;
  const int part = g.nparts == 2 && int64_t(blockIdx.x) >= half ? 1 : 0;
  const int64_t t0 = ((int64_t(blockIdx.x) - part * half) * (blockDim.x / kWave) +
                      __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave)) * CH;
  const char* src = part ? g.src1 : g.src0;
  char* dst = part ? g.dst1 : g.dst0;
  // Branch-free up to the row loads (a wave past the last token runs with
  // every row predicated off): each branch would start a new block and
  // split the argument and lookup loads into dependent rounds.
  QScale qs;
  {
    const float sv = *(g.scale ? g.scale : reinterpret_cast<const float*>(g.cu));
    qs.s = g.scale ? sv : 1.0f;
    qs.r = 0.0f;
    qs.fast = false;
    qs.neg = 0u;
  }

  // Sequence lookup without a chain of dependent loads.  The lanes hold a
  // window of 64 sequences k = wbase + lane: cu[k], cu[k+1] and seq_starts[k]
  // (clamped loads, lanes past the batch hold an end of INT32_MAX).  Token t
  // belongs to sequence wbase + n, n = the number of window entries with
  // cu[k+1] <= t (a ballot); its cu[b] and start come from lane n.  The first
  // window is loaded unconditionally; a batch of more than 64 sequences whose
  // token lies beyond it places the window with one 64-wide probe of cu[64j].
  // A later token of the chunk past the window takes the scalar walk.
  const int32_t* sp = g.starts ? g.starts : g.cu;
  const int64_t last = g.batch > 0 ? g.batch - 1 : 0;
  int64_t wbase = 0;
  int64_t kw = lane;
  int64_t cu_lo = g.cu[kw < g.batch ? kw : g.batch];
  int64_t cu_hi = g.cu[kw < g.batch ? kw + 1 : g.batch];
  int32_t st = sp[kw < last ? kw : last];
  if (g.batch > kWave && t0 >= int64_t(__builtin_amdgcn_readlane(int(cu_hi), kWave - 1))) {
    const int64_t k = (int64_t(lane) + 1) * kWave;
    const int64_t c = g.cu[k <= g.batch ? k : g.batch];
    wbase = int64_t(__popcll(__ballot(k <= g.batch && c <= t0))) * kWave;
    kw = wbase + lane;
    cu_lo = g.cu[kw < g.batch ? kw : g.batch];
    cu_hi = g.cu[kw < g.batch ? kw + 1 : g.batch];
    st = sp[kw < last ? kw : last];
  }
  if (kw >= g.batch) cu_hi = INT32_MAX;
  if (!g.starts) st = 0;
  const int64_t cu0 = g.cu[0];

  int64_t bseq[CH], pos[CH];
  int nwin[CH];
  bool slow = false;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int64_t t = t0 + c;
    const int n = __popcll(__ballot(cu_hi <= t));
    nwin[c] = n;
    slow |= n == kWave;
    const int nl = n < kWave ? n : kWave - 1;
    bseq[c] = wbase + n;
    pos[c] = int64_t(__builtin_amdgcn_readlane(st, nl)) + t - int64_t(__builtin_amdgcn_readlane(int(cu_lo), nl));
  }
  if (slow) {  // a token of this chunk lies past the window: walk on from its end
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (nwin[c] != kWave) continue;
      const int64_t t = t0 + c;
      int64_t b = wbase + kWave;
      while (b < g.batch && t >= int64_t(g.cu[b + 1])) ++b;
      bseq[c] = b;
      pos[c] = b < g.batch ? (g.starts ? int64_t(g.starts[b]) : 0) + t - int64_t(g.cu[b]) : 0;
    }
  }

  // Block-table reads through an always-valid pointer, the value passed
  // through readfirstlane before the select: a select between a loaded value
  // and a constant makes LLVM put the load behind a branch, and the branches
  // would split the CH reads into dependent rounds.
  __amdgpu_buffer_rsrc_t rin[CH], rout[CH];
  const uint32_t in_bytes = uint32_t(g.row_vecs) * C::IN_B;
  const uint32_t out_bytes = uint32_t(g.row_vecs) * C::OUT_B;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int64_t t = t0 + c;
    const int64_t p = pos[c];
    int64_t page, off;
    if (POW2) {
      page = p >> g.bs_shift;
      off = p & ((int64_t(1) << g.bs_shift) - 1);
    } else {
      page = p / g.block_size;
      off = p - page * g.block_size;
    }
    const bool wr = t < g.num_tokens && bseq[c] < g.batch && t >= cu0;
    const bool look = wr && p >= 0 && page < g.bt_stride;
    const int32_t* bp = look ? g.block_table + bseq[c] * g.bt_stride + page : g.cu;
    const int64_t v = __builtin_amdgcn_readfirstlane(*bp);
    const int64_t blk = look ? v : int64_t(-1);
    const bool rd = blk >= 0 && blk < g.num_blocks;
    // rows that must not be read come back as zeros; rows past the batch are
    // not written
    rin[c] = make_rsrc(src + blk * g.blk_stride + off * g.page_stride, rd ? in_bytes : 0u);
    rout[c] = make_rsrc(dst + t * g.dst_stride, wr ? out_bytes : 0u);
  }

  const int total = g.row_vecs;
  for (int base = 0; base < total; base += kWave * U) {
    typename C::In v[CH][U];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        v[c][u] = BufIO<C::IN_B>::load(rin[c], uint32_t(base + u * kWave + lane) * C::IN_B);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        BufIO<C::OUT_B>::store(C::apply(v[c][u], qs), rout[c], uint32_t(base + u * kWave + lane) * C::OUT_B);
    }
  }
}

// Workgroups of `wpb` waves for chunks of `ch` tokens: the same number per
// part (paged_gather_kernel splits the grid in halves between K and V).
inline int64_t gather_grid(const GatherGeom& g, int ch, int wpb) {
  return ceil_div(ceil_div(g.num_tokens, ch), wpb) * g.nparts;
}

template <class C, bool POW2>
void launch_gather_pow2(const GatherGeom& g, hipStream_t st) {
  if (g.num_tokens < 4096) {
    const int threads = g.num_tokens <= 1024 ? 64 : 256;
    hipLaunchKernelGGL((paged_gather_kernel<C, 1, 2, POW2>), dim3(gather_grid(g, 1, threads / kWave)),
                       dim3(threads), 0, st, g);
  } else {
    // About 2 KiB of cache per wave: one token of a row over 64 vectors (two
    // vectors per lane, looping beyond), two tokens of a 1 KiB row, four of a
    // smaller one.  Measured on config 3's 1 KiB rows: 118.5 us at two tokens
    // per wave, 123 at four, 133 at sixteen, 135 at one (parts interleaved);
    // with the parts in grid halves 116.5 at two, 121.7 at four, 135 at one.
    const int64_t in_row = int64_t(g.row_vecs) * C::IN_B;
    if (g.row_vecs > kWave)
      hipLaunchKernelGGL((paged_gather_kernel<C, 1, 2, POW2>), dim3(gather_grid(g, 1, 4)), dim3(256), 0, st, g);
    else if (in_row >= 1024)
      hipLaunchKernelGGL((paged_gather_kernel<C, 2, 1, POW2>), dim3(gather_grid(g, 2, 4)), dim3(256), 0, st, g);
    else
      hipLaunchKernelGGL((paged_gather_kernel<C, 4, 1, POW2>), dim3(gather_grid(g, 4, 4)), dim3(256), 0, st, g);
  }
}

template <class C>
int launch_gather(const GatherGeom& g, hipStream_t st) {
  if (g.bs_shift >= 0)
    launch_gather_pow2<C, true>(g, st);
  else
    launch_gather_pow2<C, false>(g, st);
  return check_launch("paged_gather_kernel launch");
}

int dispatch_gather(int cache_dt, int out_dt, int elems, const GatherGeom& g, hipStream_t st) {
  if (cache_dt == out_dt) {
    switch (elems * dtype_size(cache_dt)) {
      case 16: return launch_gather<CopyConv<16>>(g, st);
      case 8: return launch_gather<CopyConv<8>>(g, st);
      case 4: return launch_gather<CopyConv<4>>(g, st);
      case 2: return launch_gather<CopyConv<2>>(g, st);
      case 1: return launch_gather<CopyConv<1>>(g, st);
    }
    return fail(PSK_E_ARG, "internal: bad copy vector width");
  }
  if (cache_dt != PSK_DTYPE_FP8_E4M3FN) return fail(PSK_E_DTYPE, "output dtype must equal the cache dtype unless the cache is fp8");
#define PSK_DEQ_CASES(DT)                                         \
  switch (elems) {                                                \
    case 8: return launch_gather<DequantConv<DT, 8>>(g, st);      \
    case 4: return launch_gather<DequantConv<DT, 4>>(g, st);      \
    case 2: return launch_gather<DequantConv<DT, 2>>(g, st);      \
    case 1: return launch_gather<DequantConv<DT, 1>>(g, st);      \
  }                                                               \
  return fail(PSK_E_ARG, "internal: bad dequant vector width");
  switch (out_dt) {
    case PSK_DTYPE_BF16: { PSK_DEQ_CASES(PSK_DTYPE_BF16) }
    case PSK_DTYPE_F16: { PSK_DEQ_CASES(PSK_DTYPE_F16) }
    case PSK_DTYPE_F32: {
      switch (elems) {
        case 4: return launch_gather<DequantConv<PSK_DTYPE_F32, 4>>(g, st);
        case 2: return launch_gather<DequantConv<PSK_DTYPE_F32, 2>>(g, st);
        case 1: return launch_gather<DequantConv<PSK_DTYPE_F32, 1>>(g, st);
      }
      return fail(PSK_E_ARG, "internal: bad dequant vector width");
    }
  }
#undef PSK_DEQ_CASES
  return fail(PSK_E_DTYPE, "fp8 gather output must be bf16, fp16 or fp32");
}

// ----------------------------------------------------------------------------
// copy_blocks: one workgroup per (pair, layer) slab on a 2-D grid
// ----------------------------------------------------------------------------

// Each wave copies contiguous pieces of 64*U vectors (16 KiB at 16-byte
// vectors): a wave's loads then fall in one stretch of DRAM pages instead of
// U stretches a workgroup-width apart, which is worth 10% on random 64 KiB
// slabs.  (pair, layer) come straight from the 2-D grid, so the loads wait
// only for the two mapping entries.  The launch caps residency through its
// dynamic LDS size (see copy_blocks_lds), which the kernel never touches.
template <int B, int U>
__global__ void __launch_bounds__(256) copy_blocks_kernel(char* cache, int64_t layer_stride, int64_t block_stride,
                                                          int64_t block_bytes, int64_t num_blocks,
                                                          const int64_t* mapping) {
  using V = typename VecT<B>::T;
  const int64_t pair = blockIdx.x;
  const int64_t layer = blockIdx.y;
  const int64_t s = mapping[2 * pair];
  const int64_t d = mapping[2 * pair + 1];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return;
  const V* src = reinterpret_cast<const V*>(cache + layer * layer_stride + s * block_stride);
  V* dst = reinterpret_cast<V*>(cache + layer * layer_stride + d * block_stride);
  const int64_t nvec = block_bytes / B;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t piece = int64_t(kWave) * U;
  const int64_t step = piece * (blockDim.x / kWave);
  for (int64_t base = (threadIdx.x / kWave) * piece; base < nvec; base += step) {
    V v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * kWave + lane;
      if (i < nvec) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * kWave + lane;
      if (i < nvec) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

// LDS bytes per CU of the current device (0 if unknown), cached per device.
int64_t lds_per_cu() {
  static std::mutex mu;
  static std::map<int, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess) v = 0;
  cache[dev] = v;
  return v;
}

// Dynamic LDS that leaves room for exactly `per_cu` resident workgroups.
// Slabs of 64 KiB and more run best with three 4-wave workgroups per CU
// (measured on config 5a's random 64 KiB slabs: 6.27 TB/s against 6.08 at the
// register-limited occupancy, 5.83 at two); smaller slabs gain nothing from a
// cap and run uncapped.
int64_t copy_blocks_lds(int64_t block_bytes, int waves) {
  if (waves < 4 || block_bytes < 65536) return 0;
  const int64_t lds = lds_per_cu();
  const int per_cu = 3;
  if (lds <= 0) return 0;
  return lds / (per_cu + 1) + 1024;
}

// ----------------------------------------------------------------------------
// amax -> scale (two launches: partial maxima, then one workgroup reduces them;
// graph-safe, nothing to clear between calls)
// ----------------------------------------------------------------------------

constexpr int kAmaxMaxBlocks = 1024;
constexpr int64_t kAmaxWsLen = 2 * int64_t(kAmaxMaxBlocks);

}  // namespace

// Scratch of psk_kv_amax_scale_noalloc: the partial maxima of two tensors,
// kAmaxMaxBlocks each (8 KiB per GPU, held until the process ends).  Host code
// never uses this name as an address: each device's copy is reached through
// the pointer amax_scratch() obtains from hipGetSymbolAddress.
static __device__ __align__(256) uint32_t scratch[kAmaxWsLen];

namespace {

// This device's address of `scratch`, looked up once per device (with that
// device current) and kept; returns a status.
int amax_scratch(uint32_t** out) {
  static std::mutex mu;
  static std::map<int, uint32_t*> ptrs;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(mu);
  auto it = ptrs.find(dev);
  if (it == ptrs.end()) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(PSK_E_ARG, "hipGetSymbolAddress(scratch) returned NULL");
    it = ptrs.emplace(dev, static_cast<uint32_t*>(p)).first;
  }
  *out = it->second;
  return PSK_OK;
}

struct AmaxArgs {
  const char* x0;
  const char* x1;
  int64_t rows;
  int64_t row_vecs;
  int32_t tpr_shift;  // strided rows: log2(threads per row); rows == 1: unused
  int64_t stride0;  // bytes
  int64_t stride1;  // bytes
  float qmax;
  float* scale_out;
  float* amax_out;
  uint32_t* ws;
};

// |x| as the bit pattern of a non-negative float; NaN -> 0 so it never wins.
template <int DT> __device__ __forceinline__ uint32_t abs_bits(typename Elt<DT>::Bits b);
template <> __device__ __forceinline__ uint32_t abs_bits<PSK_DTYPE_BF16>(uint16_t b) {
  const uint32_t a = b & 0x7FFFu;
  return a > 0x7F80u ? 0u : a << 16;
}
template <> __device__ __forceinline__ uint32_t abs_bits<PSK_DTYPE_F16>(uint16_t b) {
  const float f = __builtin_fabsf(float(__builtin_bit_cast(_Float16, b)));
  return __builtin_isnan(f) ? 0u : __float_as_uint(f);
}
template <> __device__ __forceinline__ uint32_t abs_bits<PSK_DTYPE_F32>(uint32_t b) {
  const uint32_t a = b & 0x7FFFFFFFu;
  return a > 0x7F800000u ? 0u : a;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t m, uint32_t* red) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const uint32_t o = uint32_t(__shfl_xor(int(m), off, kWave));
    m = o > m ? o : m;
  }
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < int(blockDim.x / kWave); ++i) m = red[i] > m ? red[i] : m;
  }
  return m;  // valid in thread 0
}

template <int DT, int B>
__global__ void __launch_bounds__(256) amax_partial_kernel(AmaxArgs a) {
  using Bits = typename Elt<DT>::Bits;
  constexpr int E = B / int(sizeof(Bits));
  using V = typename VecT<B>::T;
  __shared__ uint32_t red[4];
  const int j = blockIdx.y;
  const char* x = j ? a.x1 : a.x0;
  const int64_t stride = j ? a.stride1 : a.stride0;
  uint32_t m = 0;
  auto take = [&](const char* p) {
    const V v = vload_nt<B>(p);
    Bits e[E];
    __builtin_memcpy(e, &v, sizeof(v));
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const uint32_t q = abs_bits<DT>(e[k]);
      m = q > m ? q : m;
    }
  };
  if (a.rows == 1) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < a.row_vecs;
         i += int64_t(gridDim.x) * blockDim.x)
      take(x + i * B);
  } else {
    // 2^tpr_shift threads per row, 256 >> tpr_shift rows per workgroup pass
    const int rpp = int(blockDim.x) >> a.tpr_shift;
    const int64_t rsub = threadIdx.x >> a.tpr_shift;
    const int64_t col0 = threadIdx.x & ((1 << a.tpr_shift) - 1);
    for (int64_t r = int64_t(blockIdx.x) * rpp + rsub; r < a.rows; r += int64_t(gridDim.x) * rpp)
      for (int64_t c = col0; c < a.row_vecs; c += (int64_t(1) << a.tpr_shift)) take(x + r * stride + c * B);
  }
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) a.ws[int64_t(j) * kAmaxMaxBlocks + blockIdx.x] = m;
}

// One workgroup: max over the partials of each tensor, then the scale.  A
// second launch instead of a last-workgroup finish: device-scope atomics and
// release fences cost more on MI355X than a kernel boundary.
__global__ void __launch_bounds__(256) amax_finalize_kernel(AmaxArgs a, int nparts, int ntensors) {
  __shared__ uint32_t red[4];
  for (int j = 0; j < ntensors; ++j) {
    uint32_t m = 0;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
      const uint32_t q = a.ws[int64_t(j) * kAmaxMaxBlocks + i];
      m = q > m ? q : m;
    }
    m = block_max_u32(m, red);
    if (threadIdx.x == 0) {
      const float amax = __uint_as_float(m);
      a.scale_out[j] = amax > 0.0f ? amax / a.qmax : 1.0f;
      if (a.amax_out) a.amax_out[j] = amax;
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------
// graph static metadata: one launch refreshes every static field
// ----------------------------------------------------------------------------

// The captured decode step reads fixed buffers; before each replay they take
// the live step's metadata, and with a padded batch (bsz < cg_bsz) the rows
// past the batch are set so that padded graph rows never write the cache and
// the readers see empty sequences.  One thread per element of the union of
// the regions, grid-stride: no memset node, so the refresh itself may also be
// captured.
struct GraphMeta {
  const int32_t* src_pt;  // [bsz, width] at src_pt_stride
  const int64_t* src_slots;
  const int32_t* src_lq;
  const int32_t* src_lkv;
  const int32_t* src_cu;  // [bsz + 1]
  int32_t* dst_pt;        // [max_bsz, >= width] at dst_pt_stride
  int64_t* dst_slots;     // [slot_cap]
  int32_t* dst_lq;
  int32_t* dst_lkv;
  int32_t* dst_cu;        // [max_bsz + 1]
  int64_t src_pt_stride, dst_pt_stride;
  int64_t bsz, width, n_slots;
  int64_t pt_rows;        // bsz, or max_bsz when padding
  int64_t slot_end;       // n_slots, or slot_cap when padding
  int64_t len_end;        // bsz, or max_bsz when padding
  int32_t pad_q_len;
  // ends of the regions in the flattened index space
  int64_t e_pt, e_slot, e_lq, e_lkv, e_cu;
};

__global__ void __launch_bounds__(256) graph_meta_refresh_kernel(GraphMeta m) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < m.e_cu; i += stride) {
    if (i < m.e_pt) {
      const int64_t r = i / m.width, c = i - r * m.width;
      m.dst_pt[r * m.dst_pt_stride + c] = r < m.bsz ? m.src_pt[r * m.src_pt_stride + c] : 0;
    } else if (i < m.e_slot) {
      const int64_t k = i - m.e_pt;
      m.dst_slots[k] = k < m.n_slots ? m.src_slots[k] : int64_t(-1);
    } else if (i < m.e_lq) {
      const int64_t k = i - m.e_slot;
      m.dst_lq[k] = k < m.bsz ? m.src_lq[k] : m.pad_q_len;
    } else if (i < m.e_lkv) {
      const int64_t k = i - m.e_lq;
      m.dst_lkv[k] = k < m.bsz ? m.src_lkv[k] : 0;
    } else {
      const int64_t k = i - m.e_lkv;
      m.dst_cu[k] = k <= m.bsz ? m.src_cu[k] : m.src_cu[m.bsz] + int32_t(k - m.bsz) * m.pad_q_len;
    }
  }
}

// ----------------------------------------------------------------------------
// swap: blit kernel over (view, page) units reading/writing mapped host memory
// ----------------------------------------------------------------------------

struct SwapView {
  uint64_t src;
  uint64_t dst;
  uint64_t bpb;
};

// One wave per (page, view) unit, grid-stride over units; each wave moves its
// page in 64 x B x U byte steps.  Wave granularity keeps small pages (4-16 KiB)
// from idling most of a workgroup, and the page-id tables are read from device
// memory (staged there by one H2D copy) rather than over the host link.
template <int B, int U>
__global__ void __launch_bounds__(256) blit_pages_kernel(const SwapView* views, const int64_t* src_pages,
                                                         const int64_t* dst_pages, int64_t num_views,
                                                         int64_t num_pages) {
  using V = typename VecT<B>::T;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves = int64_t(gridDim.x) * 4;
  const int64_t units = num_views * num_pages;
  for (int64_t unit = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
       unit < units; unit += waves) {
    const int64_t k = unit / num_views;
    const int64_t vi = unit - k * num_views;
    const SwapView view = views[vi];
    const char* src = reinterpret_cast<const char*>(view.src + uint64_t(src_pages[k]) * view.bpb);
    char* dst = reinterpret_cast<char*>(view.dst + uint64_t(dst_pages[k]) * view.bpb);
    const int64_t nvec = int64_t(view.bpb) / B;
    for (int64_t base = 0; base < nvec; base += kWave * U) {
      V v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = base + u * kWave + lane;
        if (i < nvec) v[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(src) + i);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = base + u * kWave + lane;
        if (i < nvec) __builtin_nontemporal_store(v[u], reinterpret_cast<V*>(dst) + i);
      }
    }
  }
}

// Stable LSD radix sort of indices by non-negative key, 11-bit digits, only as
// many passes as the largest key needs.  Keys below 2^32 travel packed with
// their index in one uint64 (key << 32 | index), so every pass is a sequential
// sweep; larger keys fall back to sorting indices through the key array.
void radix_order(const int64_t* key, int64_t n, std::vector<uint32_t>& order) {
  uint64_t maxk = 0;
  for (int64_t i = 0; i < n; ++i) maxk |= uint64_t(key[i]);
  order.resize(size_t(n));
  if (maxk < (uint64_t(1) << 32)) {
    std::vector<uint64_t> a(static_cast<size_t>(n)), b(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) a[size_t(i)] = (uint64_t(key[i]) << 32) | uint64_t(i);
    for (int shift = 32; shift < 64 && (maxk >> (shift - 32)) != 0; shift += 11) {
      size_t count[2049] = {0};
      for (int64_t i = 0; i < n; ++i) ++count[((a[size_t(i)] >> shift) & 2047) + 1];
      for (int d = 0; d < 2048; ++d) count[d + 1] += count[d];
      for (int64_t i = 0; i < n; ++i) b[count[(a[size_t(i)] >> shift) & 2047]++] = a[size_t(i)];
      a.swap(b);
    }
    for (int64_t i = 0; i < n; ++i) order[size_t(i)] = uint32_t(a[size_t(i)]);
    return;
  }
  for (int64_t i = 0; i < n; ++i) order[size_t(i)] = uint32_t(i);
  std::vector<uint32_t> tmp(static_cast<size_t>(n));
  for (int shift = 0; shift < 64 && (maxk >> shift) != 0; shift += 11) {
    size_t count[2049] = {0};
    for (int64_t i = 0; i < n; ++i) ++count[((uint64_t(key[order[size_t(i)]]) >> shift) & 2047) + 1];
    for (int d = 0; d < 2048; ++d) count[d + 1] += count[d];
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t o = order[size_t(i)];
      tmp[count[(uint64_t(key[o]) >> shift) & 2047]++] = o;
    }
    order.swap(tmp);
  }
}

int64_t staging_bytes(int64_t num_views, int64_t num_pages) {
  return num_views * int64_t(sizeof(SwapView)) + 2 * num_pages * int64_t(sizeof(int64_t)) + 64;
}

// ----------------------------------------------------------------------------
// XXH64 (Yann Collet's published xxHash64 specification, seed 0), host code.
// The prefix cache keys every full page by the digest of the previous page's
// key (8 bytes, little endian) followed by the page's token bytes.
// ----------------------------------------------------------------------------

constexpr uint64_t kXP1 = 0x9E3779B185EBCA87ull;
constexpr uint64_t kXP2 = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kXP3 = 0x165667B19E3779F9ull;
constexpr uint64_t kXP4 = 0x85EBCA77C2B2AE63ull;
constexpr uint64_t kXP5 = 0x27D4EB2F165667C5ull;

inline uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }

inline uint64_t load_le64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}

inline uint64_t load_le32(const uint8_t* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}

inline uint64_t xxh_lane(uint64_t acc, uint64_t lane) { return rotl64(acc + lane * kXP2, 31) * kXP1; }

inline uint64_t xxh_fold(uint64_t h, uint64_t acc) { return (h ^ xxh_lane(0, acc)) * kXP1 + kXP4; }

uint64_t xxh64(const uint8_t* p, size_t n) {
  const uint8_t* const end = p + n;
  uint64_t h;
  if (n >= 32) {
    uint64_t a0 = kXP1 + kXP2, a1 = kXP2, a2 = 0, a3 = uint64_t(0) - kXP1;
    for (; end - p >= 32; p += 32) {
      a0 = xxh_lane(a0, load_le64(p));
      a1 = xxh_lane(a1, load_le64(p + 8));
      a2 = xxh_lane(a2, load_le64(p + 16));
      a3 = xxh_lane(a3, load_le64(p + 24));
    }
    h = rotl64(a0, 1) + rotl64(a1, 7) + rotl64(a2, 12) + rotl64(a3, 18);
    h = xxh_fold(xxh_fold(xxh_fold(xxh_fold(h, a0), a1), a2), a3);
  } else {
    h = kXP5;
  }
  h += uint64_t(n);
  for (; end - p >= 8; p += 8) h = rotl64(h ^ xxh_lane(0, load_le64(p)), 27) * kXP1 + kXP4;
  if (end - p >= 4) {
    h = rotl64(h ^ (load_le32(p) * kXP1), 23) * kXP2 + kXP3;
    p += 4;
  }
  for (; p < end; ++p) h = rotl64(h ^ (uint64_t(*p) * kXP5), 11) * kXP1;
  h ^= h >> 33;
  h *= kXP2;
  h ^= h >> 29;
  h *= kXP3;
  h ^= h >> 32;
  return h;
}

// XXH64 of le64(prefix) || data[0, nbytes), or of the data alone without a prefix.
// `buf` holds 8 + nbytes bytes of room.
uint64_t keyed_digest(const uint8_t* data, size_t nbytes, uint64_t prefix, bool has_prefix, uint8_t* buf) {
  if (!has_prefix) return xxh64(data, nbytes);
  memcpy(buf, &prefix, 8);  // the host is little endian (x86-64)
  memcpy(buf + 8, data, nbytes);
  return xxh64(buf, nbytes + 8);
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================

extern "C" {

const char* psk_last_error(void) { return g_err; }

int psk_abi_version(void) { return 1; }

}  // extern "C"

namespace {

// psk_reshape_and_cache's body; fin (FP8 only): finish the amax scales in the
// append (kNeedScales when the shape does not take it: nothing launched).
int append_kv(const void* key, const void* value, void* key_cache, void* value_cache, const int64_t* slot_mapping,
              int64_t num_tokens, int64_t num_heads, int64_t head_size, int64_t block_size, int64_t num_blocks,
              int64_t key_stride, int64_t value_stride, const int64_t* kc, const int64_t* vc, int in_dtype,
              int cache_dtype, const float* k_scale, const float* v_scale, hipStream_t stream,
              const AmaxFinish* fin) {
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks < 0)
    return fail(PSK_E_ARG, "bad sizes: num_tokens=%lld num_heads=%lld head_size=%lld block_size=%lld num_blocks=%lld",
                (long long)num_tokens, (long long)num_heads, (long long)head_size, (long long)block_size,
                (long long)num_blocks);
  if (!kc || !vc) return fail(PSK_E_ARG, "cache stride arrays must not be NULL");
  const int in_sz = dtype_size(in_dtype), c_sz = dtype_size(cache_dtype);
  if (!in_sz || !c_sz) return fail(PSK_E_DTYPE, "unknown dtype code (in=%d cache=%d)", in_dtype, cache_dtype);
  if (in_dtype != cache_dtype && (cache_dtype != PSK_DTYPE_FP8_E4M3FN || in_dtype == PSK_DTYPE_FP8_E4M3FN))
    return fail(PSK_E_DTYPE, "cache dtype must equal the input dtype or be fp8_e4m3fn (in=%d cache=%d)", in_dtype,
                cache_dtype);
  if (in_dtype == cache_dtype && (k_scale || v_scale))
    return fail(PSK_E_ARG, "k_scale/v_scale only apply to an fp8 cache");
  if (num_tokens == 0) return PSK_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping)
    return fail(PSK_E_ARG, "NULL tensor pointer");

  const int64_t row = num_heads * head_size;
  ScatterGeom g;
  g.slots = slot_mapping;
  g.num_tokens = num_tokens;
  g.block_size = block_size;
  g.num_slots = num_blocks * block_size;
  g.bs_shift = log2_exact(block_size);
  g.nparts = 2;
  g.slice_shift = 0;

  // Heads are one contiguous run in the cache when dim stride is 1 and the head
  // stride is head_size; then a token's part is one flat row of row elements.
  const bool k_flat = kc[3] == 1 && (kc[2] == head_size || num_heads == 1);
  const bool v_flat = vc[3] == 1 && (vc[2] == head_size || num_heads == 1);
  const bool dim_contig = kc[3] == 1 && vc[3] == 1;
  int elems = 1;
  if (dim_contig) {
    std::vector<uint64_t> in_b = {uint64_t(uintptr_t(key)), uint64_t(uintptr_t(value)), uint64_t(key_stride * in_sz),
                                  uint64_t(value_stride * in_sz)};
    std::vector<uint64_t> out_b = {uint64_t(uintptr_t(key_cache)), uint64_t(uintptr_t(value_cache)),
                                   uint64_t(kc[0] * c_sz), uint64_t(kc[1] * c_sz), uint64_t(vc[0] * c_sz),
                                   uint64_t(vc[1] * c_sz)};
    if (!(k_flat && v_flat)) {
      out_b.push_back(uint64_t(kc[2] * c_sz));
      out_b.push_back(uint64_t(vc[2] * c_sz));
    }
    elems = pick_elems(in_sz, c_sz, in_b, out_b, (k_flat && v_flat) ? row : head_size);
    // Decode-sized FP8 appends are latency bound and each lane's quantization
    // is a serial chain of VALU work: four elements per lane over twice the
    // waves measured 2.22 us per config-2 append against 2.25 at eight.
    if (cache_dtype == PSK_DTYPE_FP8_E4M3FN && num_tokens < 1024 && elems > 4) elems = 4;
  }

  auto make_part = [&](const void* src, void* dst, int64_t src_stride, const int64_t* cs, const float* scale,
                       bool flat) {
    ScatterPart p;
    p.src = static_cast<const char*>(src);
    p.dst = static_cast<char*>(dst);
    p.scale = scale;
    p.src_stride = src_stride * in_sz;
    p.blk_stride = cs[0] * c_sz;
    p.page_stride = cs[1] * c_sz;
    p.dst_off = 0;
    if (dim_contig && flat && elems > 1) {
      p.nseg = 1;
      p.seg_vecs = int32_t(row / elems);
      p.seg_stride = 0;
      p.inner_stride = int64_t(elems) * c_sz;
    } else if (dim_contig) {
      p.nseg = int32_t(num_heads);
      p.seg_vecs = int32_t(head_size / elems);
      p.seg_stride = cs[2] * c_sz;
      p.inner_stride = int64_t(elems) * c_sz;
    } else {
      p.nseg = int32_t(num_heads);
      p.seg_vecs = int32_t(head_size);
      p.seg_stride = cs[2] * c_sz;
      p.inner_stride = cs[3] * c_sz;
    }
    return p;
  };
  const ScatterPart pk = make_part(key, key_cache, key_stride, kc, k_scale, k_flat);
  const ScatterPart pv = make_part(value, value_cache, value_stride, vc, v_scale, v_flat);
  return dispatch_scatter(in_dtype, cache_dtype, elems, g, pk, pv, stream, fin);
}

}  // namespace

extern "C" {

int psk_reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                          const int64_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
                          int64_t head_size, int64_t block_size, int64_t num_blocks, int64_t key_stride,
                          int64_t value_stride, const int64_t* kc, const int64_t* vc, int in_dtype,
                          int cache_dtype, const float* k_scale, const float* v_scale, void* stream) {
  begin_device_call();
  return append_kv(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_heads, head_size, block_size,
                   num_blocks, key_stride, value_stride, kc, vc, in_dtype, cache_dtype, k_scale, v_scale,
                   static_cast<hipStream_t>(stream), nullptr);
}

int psk_concat_and_cache_mla(const void* kv_c, const void* k_pe, void* kv_cache, const int64_t* slot_mapping,
                             int64_t num_tokens, int64_t key_len, int64_t value_len, int64_t kv_c_stride,
                             int64_t k_pe_stride, int64_t block_size, int64_t num_blocks,
                             int64_t cache_block_stride, int64_t cache_page_stride, int in_dtype, int cache_dtype,
                             const float* scale, void* stream) {
  begin_device_call();
  if (num_tokens < 0 || key_len <= 0 || value_len < 0 || block_size <= 0 || num_blocks < 0)
    return fail(PSK_E_ARG, "bad sizes: num_tokens=%lld key_len=%lld value_len=%lld block_size=%lld",
                (long long)num_tokens, (long long)key_len, (long long)value_len, (long long)block_size);
  const int in_sz = dtype_size(in_dtype), c_sz = dtype_size(cache_dtype);
  if (!in_sz || !c_sz) return fail(PSK_E_DTYPE, "unknown dtype code (in=%d cache=%d)", in_dtype, cache_dtype);
  if (in_dtype != cache_dtype && (cache_dtype != PSK_DTYPE_FP8_E4M3FN || in_dtype == PSK_DTYPE_FP8_E4M3FN))
    return fail(PSK_E_DTYPE, "cache dtype must equal the input dtype or be fp8_e4m3fn (in=%d cache=%d)", in_dtype,
                cache_dtype);
  if (in_dtype == cache_dtype && scale) return fail(PSK_E_ARG, "scale only applies to an fp8 cache");
  if (num_tokens == 0) return PSK_OK;
  if (!kv_c || !kv_cache || !slot_mapping || (value_len > 0 && !k_pe)) return fail(PSK_E_ARG, "NULL tensor pointer");

  std::vector<uint64_t> in_b = {uint64_t(uintptr_t(kv_c)), uint64_t(kv_c_stride * in_sz)};
  if (value_len > 0) {
    in_b.push_back(uint64_t(uintptr_t(k_pe)));
    in_b.push_back(uint64_t(k_pe_stride * in_sz));
  }
  std::vector<uint64_t> out_b = {uint64_t(uintptr_t(kv_cache)), uint64_t(cache_block_stride * c_sz),
                                 uint64_t(cache_page_stride * c_sz), uint64_t(key_len * c_sz)};
  int64_t seg = key_len;
  // the vector must also divide value_len; fold it in through the gcd
  int64_t a = key_len, b = value_len;
  while (b) { const int64_t t = a % b; a = b; b = t; }
  seg = a;
  const int elems = pick_elems(in_sz, c_sz, in_b, out_b, seg);

  ScatterGeom g;
  g.slots = slot_mapping;
  g.num_tokens = num_tokens;
  g.block_size = block_size;
  g.num_slots = num_blocks * block_size;
  g.bs_shift = log2_exact(block_size);
  g.nparts = value_len > 0 ? 2 : 1;
  g.slice_shift = 0;
  auto make_part = [&](const void* src, int64_t src_stride, int64_t len, int64_t dst_off) {
    ScatterPart p;
    p.src = static_cast<const char*>(src);
    p.dst = static_cast<char*>(kv_cache);
    p.scale = scale;
    p.src_stride = src_stride * in_sz;
    p.blk_stride = cache_block_stride * c_sz;
    p.page_stride = cache_page_stride * c_sz;
    p.dst_off = dst_off * c_sz;
    p.nseg = 1;
    p.seg_vecs = int32_t(len / elems);
    p.seg_stride = 0;
    p.inner_stride = int64_t(elems) * c_sz;
    return p;
  };
  const ScatterPart p0 = make_part(kv_c, kv_c_stride, key_len, 0);
  const ScatterPart p1 = value_len > 0 ? make_part(k_pe, k_pe_stride, value_len, key_len) : p0;
  return dispatch_scatter(in_dtype, cache_dtype, elems, g, p0, p1, static_cast<hipStream_t>(stream));
}

int psk_gather_cache(const void* src0, const void* src1, void* dst0, void* dst1, const int32_t* block_table,
                     const int32_t* cu_seq_lens, const int32_t* seq_starts, int64_t batch_size,
                     int64_t block_table_stride, int64_t num_tokens, int64_t row_len, int64_t block_size,
                     int64_t num_blocks, int64_t cache_block_stride, int64_t cache_page_stride,
                     int64_t dst_row_stride, int cache_dtype, int out_dtype, const float* scale, void* stream) {
  begin_device_call();
  if (batch_size < 0 || num_tokens < 0 || row_len <= 0 || block_size <= 0 || num_blocks < 0 ||
      block_table_stride < 0)
    return fail(PSK_E_ARG, "bad sizes: batch=%lld num_tokens=%lld row_len=%lld block_size=%lld",
                (long long)batch_size, (long long)num_tokens, (long long)row_len, (long long)block_size);
  if ((src1 == nullptr) != (dst1 == nullptr)) return fail(PSK_E_ARG, "src1 and dst1 must both be set or both NULL");
  const int c_sz = dtype_size(cache_dtype), o_sz = dtype_size(out_dtype);
  if (!c_sz || !o_sz) return fail(PSK_E_DTYPE, "unknown dtype code (cache=%d out=%d)", cache_dtype, out_dtype);
  if (cache_dtype != out_dtype && (cache_dtype != PSK_DTYPE_FP8_E4M3FN || out_dtype == PSK_DTYPE_FP8_E4M3FN))
    return fail(PSK_E_DTYPE, "out dtype must equal the cache dtype unless the cache is fp8 (cache=%d out=%d)",
                cache_dtype, out_dtype);
  if (cache_dtype == out_dtype && scale) return fail(PSK_E_ARG, "scale only applies to an fp8 -> float gather");
  if (num_tokens == 0 || batch_size == 0) return PSK_OK;
  if (!src0 || !dst0 || !block_table || !cu_seq_lens) return fail(PSK_E_ARG, "NULL tensor pointer");

  std::vector<uint64_t> in_b = {uint64_t(uintptr_t(src0)), uint64_t(cache_block_stride * c_sz),
                                uint64_t(cache_page_stride * c_sz)};
  std::vector<uint64_t> out_b = {uint64_t(uintptr_t(dst0)), uint64_t(dst_row_stride * o_sz)};
  if (src1) {
    in_b.push_back(uint64_t(uintptr_t(src1)));
    out_b.push_back(uint64_t(uintptr_t(dst1)));
  }
  const int elems = pick_elems(c_sz, o_sz, in_b, out_b, row_len);

  GatherGeom g;
  g.src0 = static_cast<const char*>(src0);
  g.src1 = static_cast<const char*>(src1);
  g.dst0 = static_cast<char*>(dst0);
  g.dst1 = static_cast<char*>(dst1);
  g.block_table = block_table;
  g.cu = cu_seq_lens;
  g.starts = seq_starts;
  g.scale = scale;
  g.batch = batch_size;
  g.bt_stride = block_table_stride;
  g.num_tokens = num_tokens;
  g.block_size = block_size;
  g.num_blocks = num_blocks;
  g.blk_stride = cache_block_stride * c_sz;
  g.page_stride = cache_page_stride * c_sz;
  g.dst_stride = dst_row_stride * o_sz;
  g.row_vecs = int32_t(row_len / elems);
  g.bs_shift = log2_exact(block_size);
  g.nparts = src1 ? 2 : 1;
  return dispatch_gather(cache_dtype, out_dtype, elems, g, static_cast<hipStream_t>(stream));
}

int psk_copy_blocks(void* cache, int64_t num_layers, int64_t layer_stride, int64_t block_stride,
                    int64_t block_bytes, int64_t num_blocks, const int64_t* block_mapping, int64_t num_pairs,
                    void* stream) {
  begin_device_call();
  if (num_layers < 0 || num_pairs < 0 || block_bytes < 0 || num_blocks < 0 || layer_stride < 0 ||
      block_stride < 0)
    return fail(PSK_E_ARG, "bad sizes: layers=%lld pairs=%lld block_bytes=%lld", (long long)num_layers,
                (long long)num_pairs, (long long)block_bytes);
  if (block_bytes > block_stride && num_blocks > 1)
    return fail(PSK_E_ARG, "block_bytes %lld exceeds block_stride %lld", (long long)block_bytes,
                (long long)block_stride);
  if (num_layers == 0 || num_pairs == 0 || block_bytes == 0) return PSK_OK;
  if (!cache || !block_mapping) return fail(PSK_E_ARG, "NULL pointer");
  if (num_layers > 65535) return fail(PSK_E_ARG, "num_layers %lld exceeds 65535", (long long)num_layers);
  // the grid's x extent in work-items (pairs x 256) must fit in 32 bits
  if (num_pairs > (int64_t(1) << 24)) return fail(PSK_E_ARG, "num_pairs %lld exceeds 2^24", (long long)num_pairs);
  const uint64_t vals[4] = {uint64_t(uintptr_t(cache)), uint64_t(layer_stride), uint64_t(block_stride),
                            uint64_t(block_bytes)};
  const int vb = common_align(vals, 4, 16);
  // one wave per 64*16 vectors of the slab, at most four per workgroup
  const int64_t pieces = ceil_div(block_bytes / vb, int64_t(kWave) * 16);
  const int waves = pieces >= 4 ? 4 : int(pieces);
  const dim3 grid{unsigned(num_pairs), unsigned(num_layers), 1u};
  const dim3 block{unsigned(waves * kWave), 1u, 1u};
  const size_t lds = size_t(copy_blocks_lds(block_bytes, waves));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* c = static_cast<char*>(cache);
  switch (vb) {
    case 16: hipLaunchKernelGGL((copy_blocks_kernel<16, 16>), grid, block, lds, st, c, layer_stride, block_stride, block_bytes, num_blocks, block_mapping); break;
    case 8: hipLaunchKernelGGL((copy_blocks_kernel<8, 16>), grid, block, lds, st, c, layer_stride, block_stride, block_bytes, num_blocks, block_mapping); break;
    case 4: hipLaunchKernelGGL((copy_blocks_kernel<4, 16>), grid, block, lds, st, c, layer_stride, block_stride, block_bytes, num_blocks, block_mapping); break;
    case 2: hipLaunchKernelGGL((copy_blocks_kernel<2, 16>), grid, block, lds, st, c, layer_stride, block_stride, block_bytes, num_blocks, block_mapping); break;
    default: hipLaunchKernelGGL((copy_blocks_kernel<1, 16>), grid, block, lds, st, c, layer_stride, block_stride, block_bytes, num_blocks, block_mapping); break;
  }
  return check_launch("copy_blocks_kernel launch");
}

int64_t psk_swap_staging_bytes(int64_t num_views, int64_t num_pages) { return staging_bytes(num_views, num_pages); }

int64_t psk_coalesce_runs(const int64_t* src, const int64_t* dst, int64_t n, int64_t* run_src, int64_t* run_dst,
                          int64_t* run_len) {
  g_err[0] = 0;
  if (n < 0 || n > int64_t(UINT32_MAX)) return fail(PSK_E_ARG, "page count %lld out of range", (long long)n);
  if (n == 0) return 0;
  if (!src || !dst || !run_src || !run_dst || !run_len) return fail(PSK_E_ARG, "NULL array");
  for (int64_t i = 0; i < n; ++i)
    if (src[i] < 0 || dst[i] < 0) return fail(PSK_E_RANGE, "negative page id at %lld", (long long)i);
  std::vector<uint32_t> order;
  radix_order(src, n, order);
  int64_t runs = 0;
  int64_t ps = src[order[0]], pd = dst[order[0]];
  run_src[0] = ps;
  run_dst[0] = pd;
  run_len[0] = 1;
  for (int64_t i = 1; i < n; ++i) {
    const int64_t s = src[order[size_t(i)]], d = dst[order[size_t(i)]];
    if (s == ps + 1 && d == pd + 1) {
      ++run_len[runs];
    } else {
      ++runs;
      run_src[runs] = s;
      run_dst[runs] = d;
      run_len[runs] = 1;
    }
    ps = s;
    pd = d;
  }
  return runs + 1;
}

int psk_swap_blocks(int transport, const uint64_t* src_bases, const uint64_t* dst_bases,
                    const uint64_t* bytes_per_page, int64_t num_views, const int64_t* src_start,
                    const int64_t* dst_start, const int64_t* run_len, int64_t num_runs, int64_t src_num_pages,
                    int64_t dst_num_pages, void* staging, int64_t staging_bytes_avail, void* desc_dev,
                    int64_t desc_dev_bytes, void* stream) {
  begin_device_call();
  if (num_views < 0 || num_runs < 0) return fail(PSK_E_ARG, "negative view or run count");
  if (num_views == 0 || num_runs == 0) return PSK_OK;
  if (!src_bases || !dst_bases || !bytes_per_page || !src_start || !dst_start || !run_len)
    return fail(PSK_E_ARG, "NULL descriptor array");
  int64_t pages = 0;
  for (int64_t r = 0; r < num_runs; ++r) {
    const int64_t s = src_start[r], d = dst_start[r], n = run_len[r];
    if (n <= 0) return fail(PSK_E_ARG, "run %lld has length %lld", (long long)r, (long long)n);
    if (s < 0 || s + n > src_num_pages)
      return fail(PSK_E_RANGE, "run %lld src pages [%lld, %lld) outside [0, %lld)", (long long)r, (long long)s,
                  (long long)(s + n), (long long)src_num_pages);
    if (d < 0 || d + n > dst_num_pages)
      return fail(PSK_E_RANGE, "run %lld dst pages [%lld, %lld) outside [0, %lld)", (long long)r, (long long)d,
                  (long long)(d + n), (long long)dst_num_pages);
    pages += n;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (transport == PSK_SWAP_MEMCPY) {
    for (int64_t v = 0; v < num_views; ++v) {
      for (int64_t r = 0; r < num_runs; ++r) {
        const uint64_t bpb = bytes_per_page[v];
        hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(dst_bases[v] + uint64_t(dst_start[r]) * bpb),
                                      reinterpret_cast<const void*>(src_bases[v] + uint64_t(src_start[r]) * bpb),
                                      size_t(bpb * uint64_t(run_len[r])), hipMemcpyDefault, st);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
      }
    }
    return PSK_OK;
  }
  if (transport != PSK_SWAP_BLIT) return fail(PSK_E_ARG, "unknown swap transport %d", transport);
  const int64_t need = staging_bytes(num_views, pages);
  if (!staging || staging_bytes_avail < need)
    return fail(PSK_E_WORKSPACE, "swap staging needs %lld bytes, got %lld", (long long)need,
                (long long)staging_bytes_avail);
  // Staging layout: SwapView[num_views] | int64 src_pages[pages] | int64 dst_pages[pages]
  char* base = reinterpret_cast<char*>((uintptr_t(staging) + 15) & ~uintptr_t(15));
  SwapView* views = reinterpret_cast<SwapView*>(base);
  int64_t* sp = reinterpret_cast<int64_t*>(base + num_views * int64_t(sizeof(SwapView)));
  int64_t* dp = sp + pages;
  uint64_t acc = 0;
  for (int64_t v = 0; v < num_views; ++v) {
    views[v].src = src_bases[v];
    views[v].dst = dst_bases[v];
    views[v].bpb = bytes_per_page[v];
    acc |= src_bases[v] | dst_bases[v] | bytes_per_page[v];
  }
  int64_t k = 0;
  for (int64_t r = 0; r < num_runs; ++r)
    for (int64_t i = 0; i < run_len[r]; ++i, ++k) {
      sp[k] = src_start[r] + i;
      dp[k] = dst_start[r] + i;
    }
  // Descriptors go to device memory with one async copy (the staging buffer is
  // pinned) when a device buffer is given; otherwise the kernel reads them from
  // the mapped staging buffer directly.
  const char* desc = base;
  if (desc_dev) {
    if (desc_dev_bytes < need) return fail(PSK_E_WORKSPACE, "swap device descriptors need %lld bytes, got %lld",
                                           (long long)need, (long long)desc_dev_bytes);
    const size_t used = size_t(reinterpret_cast<char*>(dp + pages) - base);
    char* dbase = reinterpret_cast<char*>((uintptr_t(desc_dev) + 15) & ~uintptr_t(15));
    hipError_t e = hipMemcpyAsync(dbase, base, used, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync (swap descriptors)");
    desc = dbase;
  }
  const SwapView* dviews = reinterpret_cast<const SwapView*>(desc);
  const int64_t* dsp = reinterpret_cast<const int64_t*>(desc + num_views * int64_t(sizeof(SwapView)));
  const int64_t* ddp = dsp + pages;
  const int64_t units = num_views * pages;
  const int64_t grid = ceil_div(units, 4) < 8192 ? ceil_div(units, 4) : 8192;
  if ((acc & 15) == 0)
    hipLaunchKernelGGL((blit_pages_kernel<16, 4>), dim3(grid), dim3(256), 0, st, dviews, dsp, ddp, num_views, pages);
  else if ((acc & 3) == 0)
    hipLaunchKernelGGL((blit_pages_kernel<4, 4>), dim3(grid), dim3(256), 0, st, dviews, dsp, ddp, num_views, pages);
  else
    hipLaunchKernelGGL((blit_pages_kernel<1, 4>), dim3(grid), dim3(256), 0, st, dviews, dsp, ddp, num_views, pages);
  return check_launch("blit_pages_kernel launch");
}

int64_t psk_build_kv_metadata(int64_t num_seqs, const uint64_t* page_table_ptrs, const int64_t* page_table_lens,
                              const int64_t* num_tokens, const int64_t* offsets, int64_t page_size, int64_t dcp_deg,
                              int64_t dcp_rank, int64_t dcp_interleave, int is_decode, int64_t row_width,
                              int32_t* page_table_out, int32_t* cu_seqlens_q_out, int32_t* lens_q_out,
                              int32_t* lens_kv_out, int64_t* slot_mapping_out, int64_t slot_capacity) {
  g_err[0] = 0;
  if (num_seqs < 0 || page_size <= 0 || dcp_deg <= 0 || dcp_rank < 0 || dcp_rank >= dcp_deg || dcp_interleave <= 0 ||
      row_width < 0 || slot_capacity < 0)
    return fail(PSK_E_ARG, "bad metadata geometry (seqs=%lld page_size=%lld dcp=%lld/%lld interleave=%lld)",
                (long long)num_seqs, (long long)page_size, (long long)dcp_rank, (long long)dcp_deg,
                (long long)dcp_interleave);
  if (dcp_deg > 1 && page_size % dcp_deg) return fail(PSK_E_ARG, "page_size must divide by the DCP degree");
  if (num_seqs && (!page_table_ptrs || !page_table_lens || !num_tokens || !offsets || !cu_seqlens_q_out ||
                   !lens_q_out || !lens_kv_out || (row_width && !page_table_out)))
    return fail(PSK_E_ARG, "NULL array");
  const int64_t phys = dcp_deg == 1 ? page_size : page_size / dcp_deg;
  const int64_t stride = dcp_interleave * dcp_deg;
  int64_t total = 0;
  cu_seqlens_q_out[0] = 0;
  for (int64_t i = 0; i < num_seqs; ++i) {
    const int64_t n = num_tokens[i], off = offsets[i], pages = page_table_lens[i];
    if (off < 0 || off > n) return fail(PSK_E_ARG, "sequence %lld: offset %lld outside [0, %lld]", (long long)i,
                                        (long long)off, (long long)n);
    if (pages > row_width) return fail(PSK_E_ARG, "sequence %lld has %lld pages, row width %lld", (long long)i,
                                       (long long)pages, (long long)row_width);
    if (n > 0 && (n - 1) / page_size >= pages)
      return fail(PSK_E_RANGE, "sequence %lld: position %lld needs page %lld of %lld", (long long)i,
                  (long long)(n - 1), (long long)((n - 1) / page_size), (long long)pages);
    const int64_t q = n - off;
    if (total + q > slot_capacity) return fail(PSK_E_WORKSPACE, "slot_mapping capacity %lld exceeded",
                                               (long long)slot_capacity);
    const int32_t* pt = reinterpret_cast<const int32_t*>(uintptr_t(page_table_ptrs[i]));
    int32_t* row = page_table_out + i * row_width;
    for (int64_t j = 0; j < pages; ++j) row[j] = pt[j];
    for (int64_t j = pages; j < row_width; ++j) row[j] = 0;
    lens_q_out[i] = int32_t(q);
    if (dcp_deg == 1) {
      lens_kv_out[i] = int32_t(n);
      int64_t* out = slot_mapping_out + total;
      for (int64_t pos = off; pos < n; ++pos) *out++ = int64_t(pt[pos / page_size]) * page_size + pos % page_size;
    } else {
      const int64_t prefix = (is_decode && q == 1) ? n : off;
      int64_t kv = prefix / stride * dcp_interleave;
      const int64_t rem = prefix % stride;
      if (rem >= (dcp_rank + 1) * dcp_interleave) kv += dcp_interleave;
      else if (rem >= dcp_rank * dcp_interleave) kv += rem % dcp_interleave;
      lens_kv_out[i] = int32_t(kv);
      int64_t* out = slot_mapping_out + total;
      for (int64_t pos = off; pos < n; ++pos) {
        if ((pos / dcp_interleave) % dcp_deg == dcp_rank) {
          const int64_t local = pos % dcp_interleave + pos / stride * dcp_interleave;
          *out++ = int64_t(pt[pos / page_size]) * phys + local % phys;
        } else {
          *out++ = -1;
        }
      }
    }
    total += q;
    cu_seqlens_q_out[i + 1] = int32_t(total);
  }
  return total;
}

int psk_refresh_graph_metadata(const int32_t* src_page_table, int64_t src_page_table_stride,
                                const int64_t* src_slot_mapping, const int32_t* src_lens_q,
                                const int32_t* src_lens_kv, const int32_t* src_cu_seqlens_q, int64_t bsz,
                                int64_t width, int64_t num_slots, int32_t* dst_page_table,
                                int64_t dst_page_table_stride, int64_t dst_page_table_width,
                                int64_t* dst_slot_mapping, int64_t slot_capacity, int32_t* dst_lens_q,
                                int32_t* dst_lens_kv, int32_t* dst_cu_seqlens_q, int64_t max_bsz, int64_t cg_bsz,
                                int32_t pad_q_len, void* stream) {
  begin_device_call();
  if (bsz < 0 || width < 0 || num_slots < 0 || max_bsz < 0 || slot_capacity < 0)
    return fail(PSK_E_ARG, "negative graph metadata size");
  if (bsz > cg_bsz || cg_bsz > max_bsz)
    return fail(PSK_E_ARG, "batch %lld does not fit the graph batch %lld of the static buffers (%lld rows)",
                (long long)bsz, (long long)cg_bsz, (long long)max_bsz);
  if (width > dst_page_table_width)
    return fail(PSK_E_ARG, "page table width %lld exceeds the static width %lld", (long long)width,
                (long long)dst_page_table_width);
  if (num_slots > slot_capacity)
    return fail(PSK_E_ARG, "%lld slots exceed the static slot_mapping capacity %lld", (long long)num_slots,
                (long long)slot_capacity);
  if (src_page_table_stride < width || dst_page_table_stride < dst_page_table_width)
    return fail(PSK_E_ARG, "page table row stride smaller than its width");
  const bool pad = bsz != cg_bsz;
  if (pad && pad_q_len < 0) return fail(PSK_E_ARG, "negative pad_q_len");
  if ((bsz && (!src_lens_q || !src_lens_kv)) || !src_cu_seqlens_q || !dst_cu_seqlens_q ||
      (num_slots && !src_slot_mapping) || (bsz * width && !src_page_table) ||
      ((pad ? max_bsz : bsz) * width && !dst_page_table) || ((pad ? slot_capacity : num_slots) && !dst_slot_mapping) ||
      ((pad ? max_bsz : bsz) && (!dst_lens_q || !dst_lens_kv)))
    return fail(PSK_E_ARG, "NULL metadata pointer");
  GraphMeta m;
  m.src_pt = src_page_table;
  m.src_slots = src_slot_mapping;
  m.src_lq = src_lens_q;
  m.src_lkv = src_lens_kv;
  m.src_cu = src_cu_seqlens_q;
  m.dst_pt = dst_page_table;
  m.dst_slots = dst_slot_mapping;
  m.dst_lq = dst_lens_q;
  m.dst_lkv = dst_lens_kv;
  m.dst_cu = dst_cu_seqlens_q;
  m.src_pt_stride = src_page_table_stride;
  m.dst_pt_stride = dst_page_table_stride;
  m.bsz = bsz;
  m.width = width;
  m.n_slots = num_slots;
  m.pt_rows = pad ? max_bsz : bsz;
  m.slot_end = pad ? slot_capacity : num_slots;
  m.len_end = pad ? max_bsz : bsz;
  m.pad_q_len = pad_q_len;
  m.e_pt = m.pt_rows * width;
  m.e_slot = m.e_pt + m.slot_end;
  m.e_lq = m.e_slot + m.len_end;
  m.e_lkv = m.e_lq + m.len_end;
  m.e_cu = m.e_lkv + m.len_end + 1;
  const int64_t blocks = ceil_div(m.e_cu, 256) < 1024 ? ceil_div(m.e_cu, 256) : 1024;
  hipLaunchKernelGGL(graph_meta_refresh_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), m);
  return check_launch("graph_meta_refresh_kernel launch");
}

int64_t psk_build_next_decode_metadata(int64_t num_seqs, const uint64_t* page_table_ptrs,
                                       const int64_t* page_table_lens, const int64_t* positions,
                                       const int32_t* lens_kv_prev, int64_t page_size, int64_t dcp_deg,
                                       int64_t dcp_rank, int64_t dcp_interleave, int64_t* slot_mapping_out,
                                       int32_t* lens_kv_out) {
  g_err[0] = 0;
  if (num_seqs < 0 || page_size <= 0 || dcp_deg <= 0 || dcp_rank < 0 || dcp_rank >= dcp_deg || dcp_interleave <= 0)
    return fail(PSK_E_ARG, "bad decode metadata geometry (seqs=%lld page_size=%lld dcp=%lld/%lld interleave=%lld)",
                (long long)num_seqs, (long long)page_size, (long long)dcp_rank, (long long)dcp_deg,
                (long long)dcp_interleave);
  if (dcp_deg > 1 && page_size % dcp_deg) return fail(PSK_E_ARG, "page_size must divide by the DCP degree");
  if (num_seqs && (!page_table_ptrs || !page_table_lens || !positions || !lens_kv_prev || !slot_mapping_out ||
                   !lens_kv_out))
    return fail(PSK_E_ARG, "NULL array");
  const int64_t phys = dcp_deg == 1 ? page_size : page_size / dcp_deg;
  const int64_t stride = dcp_interleave * dcp_deg;
  for (int64_t i = 0; i < num_seqs; ++i) {
    const int64_t pos = positions[i];
    if (pos < 0 || pos / page_size >= page_table_lens[i])
      return fail(PSK_E_RANGE, "sequence %lld: position %lld needs page %lld of %lld", (long long)i, (long long)pos,
                  (long long)(pos < 0 ? -1 : pos / page_size), (long long)page_table_lens[i]);
    const int32_t* pt = reinterpret_cast<const int32_t*>(uintptr_t(page_table_ptrs[i]));
    const int64_t page = pt[pos / page_size];
    if (dcp_deg == 1) {
      slot_mapping_out[i] = page * page_size + pos % page_size;
      lens_kv_out[i] = lens_kv_prev[i] + 1;
    } else if ((pos / dcp_interleave) % dcp_deg == dcp_rank) {
      const int64_t local = pos % dcp_interleave + pos / stride * dcp_interleave;
      slot_mapping_out[i] = page * phys + local % phys;
      lens_kv_out[i] = lens_kv_prev[i] + 1;
    } else {
      slot_mapping_out[i] = -1;
      lens_kv_out[i] = lens_kv_prev[i];
    }
  }
  return num_seqs;
}

int64_t psk_kv_amax_workspace_len(void) { return kAmaxWsLen; }

}  // extern "C"

namespace {

// psk_kv_amax_scale's first launch (its arguments checked by the caller): the
// partial maxima into `workspace`; *args and *blocks_out describe them for the
// finish (amax_finalize_kernel, or an append that finishes them itself).
int amax_partials(const void* x0, const void* x1, int64_t rows, int64_t row_len, int64_t row_stride0,
                  int64_t row_stride1, int dtype, float qmax, float* scale_out, float* amax_out, uint32_t* workspace,
                  hipStream_t st, AmaxArgs* args, int64_t* blocks_out) {
  const int sz = dtype_size(dtype);
  int64_t rws = rows, rl = row_len;
  // A contiguous tensor is one long row.
  const bool contig0 = row_stride0 == row_len, contig1 = !x1 || row_stride1 == row_len;
  if (contig0 && contig1) {
    rl = rows * row_len;
    rws = rl > 0 ? 1 : 0;
  }
  const uint64_t vals[4] = {uint64_t(uintptr_t(x0)), uint64_t(uintptr_t(x1)), uint64_t(row_stride0 * sz),
                            uint64_t(rl * sz)};
  uint64_t vals2[5] = {vals[0], vals[1], vals[2], vals[3], uint64_t(row_stride1 * sz)};
  const int vb = common_align(vals2, 5, 16);
  const int64_t row_vecs = rl * sz / vb;
  int tpr_shift = 0;
  while (tpr_shift < 8 && (int64_t(1) << tpr_shift) < row_vecs) ++tpr_shift;
  int64_t blocks;
  if (rws == 1) blocks = ceil_div(row_vecs > 0 ? row_vecs : 1, 256);
  else blocks = ceil_div(rws, int64_t(256) >> tpr_shift);
  if (blocks < 1) blocks = 1;
  if (blocks > kAmaxMaxBlocks) blocks = kAmaxMaxBlocks;
  AmaxArgs a;
  a.x0 = static_cast<const char*>(x0);
  a.x1 = static_cast<const char*>(x1 ? x1 : x0);
  a.rows = rws;
  a.row_vecs = row_vecs;
  a.tpr_shift = tpr_shift;
  a.stride0 = row_stride0 * sz;
  a.stride1 = (x1 ? row_stride1 : row_stride0) * sz;
  a.qmax = qmax;
  a.scale_out = scale_out;
  a.amax_out = amax_out;
  a.ws = workspace;
  const dim3 grid(unsigned(blocks), x1 ? 2u : 1u);
#define PSK_AMAX_LAUNCH(DT)                                                                                     \
  switch (vb) {                                                                                                 \
    case 16: hipLaunchKernelGGL((amax_partial_kernel<DT, 16>), grid, dim3(256), 0, st, a); break;               \
    case 8: hipLaunchKernelGGL((amax_partial_kernel<DT, 8>), grid, dim3(256), 0, st, a); break;                 \
    case 4: hipLaunchKernelGGL((amax_partial_kernel<DT, 4>), grid, dim3(256), 0, st, a); break;                 \
    default: hipLaunchKernelGGL((amax_partial_kernel<DT, (DT == PSK_DTYPE_F32 ? 4 : 2)>), grid, dim3(256), 0, st, a); break; \
  }
  switch (dtype) {
    case PSK_DTYPE_BF16: PSK_AMAX_LAUNCH(PSK_DTYPE_BF16) break;
    case PSK_DTYPE_F16: PSK_AMAX_LAUNCH(PSK_DTYPE_F16) break;
    case PSK_DTYPE_F32: PSK_AMAX_LAUNCH(PSK_DTYPE_F32) break;
  }
#undef PSK_AMAX_LAUNCH
  *args = a;
  *blocks_out = blocks;
  return check_launch("amax_partial_kernel launch");
}

}  // namespace

extern "C" {

int psk_kv_amax_scale(const void* x0, const void* x1, int64_t rows, int64_t row_len, int64_t row_stride0,
                      int64_t row_stride1, int dtype, float qmax, float* scale_out, float* amax_out,
                      uint32_t* workspace, int64_t workspace_len, void* stream) {
  begin_device_call();
  if (rows < 0 || row_len < 0) return fail(PSK_E_ARG, "negative size");
  const int sz = dtype_size(dtype);
  if (!sz || dtype == PSK_DTYPE_FP8_E4M3FN) return fail(PSK_E_DTYPE, "amax input must be bf16, fp16 or fp32");
  if (!(qmax > 0.0f)) return fail(PSK_E_ARG, "qmax must be positive");
  // an empty tensor (NULL data) reads nothing: its amax is 0 and its scale 1.0
  if ((!x0 && rows * row_len > 0) || !scale_out || !workspace) return fail(PSK_E_ARG, "NULL pointer");
  if (workspace_len < kAmaxWsLen)
    return fail(PSK_E_WORKSPACE, "amax workspace needs %lld uint32 words, got %lld", (long long)kAmaxWsLen,
                (long long)workspace_len);
  AmaxArgs a;
  int64_t blocks = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int st1 = amax_partials(x0, x1, rows, row_len, row_stride0, row_stride1, dtype, qmax, scale_out, amax_out,
                                workspace, st, &a, &blocks);
  if (st1 != PSK_OK) return st1;
  hipLaunchKernelGGL(amax_finalize_kernel, dim3(1), dim3(256), 0, st, a, int(blocks), x1 ? 2 : 1);
  return check_launch("amax_finalize_kernel launch");
}

int psk_kv_amax_scale_noalloc(const void* x0, const void* x1, int64_t rows, int64_t row_len, int64_t row_stride0,
                              int64_t row_stride1, int dtype, float qmax, float* scale_out, float* amax_out,
                              void* stream) {
  begin_device_call();
  uint32_t* ws = nullptr;
  const int st = amax_scratch(&ws);
  if (st != PSK_OK) return st;
  // The amax kernel writes at most kAmaxMaxBlocks partial maxima per tensor
  // whatever the input size (its grid is capped there and each thread strides
  // over the rest), so every input fits the scratch; the workspace check of
  // psk_kv_amax_scale rejects any change that would break that.
  return psk_kv_amax_scale(x0, x1, rows, row_len, row_stride0, row_stride1, dtype, qmax, scale_out, amax_out, ws,
                           kAmaxWsLen, stream);
}

int psk_reshape_and_cache_amax(const void* key, const void* value, void* key_cache, void* value_cache,
                               const int64_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
                               int64_t head_size, int64_t block_size, int64_t num_blocks, int64_t key_stride,
                               int64_t value_stride, const int64_t* kc, const int64_t* vc, int in_dtype, float qmax,
                               float* scales_out, float* amax_out, uint32_t* workspace, int64_t workspace_len,
                               void* stream) {
  begin_device_call();
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks < 0)
    return fail(PSK_E_ARG, "bad sizes: num_tokens=%lld num_heads=%lld head_size=%lld block_size=%lld num_blocks=%lld",
                (long long)num_tokens, (long long)num_heads, (long long)head_size, (long long)block_size,
                (long long)num_blocks);
  if (in_dtype != PSK_DTYPE_BF16 && in_dtype != PSK_DTYPE_F16 && in_dtype != PSK_DTYPE_F32)
    return fail(PSK_E_DTYPE, "amax-scaled append input must be bf16, fp16 or fp32 (got %d)", in_dtype);
  if (!(qmax > 0.0f)) return fail(PSK_E_ARG, "qmax must be positive");
  if (!scales_out || !workspace || !kc || !vc) return fail(PSK_E_ARG, "NULL pointer");
  if (workspace_len < kAmaxWsLen)
    return fail(PSK_E_WORKSPACE, "amax workspace needs %lld uint32 words, got %lld", (long long)kAmaxWsLen,
                (long long)workspace_len);
  const int64_t row = num_heads * head_size;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (num_tokens == 0) {  // empty K and V: scale 1.0 each, nothing to append
    int r = psk_kv_amax_scale(key, nullptr, 0, row, row, row, in_dtype, qmax, scales_out, amax_out, workspace,
                              workspace_len, stream);
    if (r != PSK_OK) return r;
    return psk_kv_amax_scale(value, nullptr, 0, row, row, row, in_dtype, qmax, scales_out + 1,
                             amax_out ? amax_out + 1 : nullptr, workspace, workspace_len, stream);
  }
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) return fail(PSK_E_ARG, "NULL tensor pointer");
  AmaxArgs a;
  int64_t blocks = 0;
  int r = amax_partials(key, value, num_tokens, row, key_stride, value_stride, in_dtype, qmax, scales_out, amax_out,
                        workspace, st, &a, &blocks);
  if (r != PSK_OK) return r;
  const AmaxFinish f{workspace, kAmaxMaxBlocks, int32_t(blocks), qmax, scales_out, amax_out};
  r = append_kv(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_heads, head_size, block_size,
                num_blocks, key_stride, value_stride, kc, vc, in_dtype, PSK_DTYPE_FP8_E4M3FN, nullptr, nullptr, st, &f);
  if (r != kNeedScales) return r;
  // a shape the fused finish does not take: finalize, then the plain append
  hipLaunchKernelGGL(amax_finalize_kernel, dim3(1), dim3(256), 0, st, a, int(blocks), 2);
  r = check_launch("amax_finalize_kernel launch");
  if (r != PSK_OK) return r;
  return append_kv(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_heads, head_size, block_size,
                   num_blocks, key_stride, value_stride, kc, vc, in_dtype, PSK_DTYPE_FP8_E4M3FN, scales_out,
                   scales_out + 1, st, nullptr);
}

int psk_host_alloc(int64_t bytes, void** ptr) {
  g_err[0] = 0;
  if (!ptr || bytes <= 0) return fail(PSK_E_ARG, "bad host allocation request (%lld bytes)", (long long)bytes);
  *ptr = nullptr;
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, size_t(bytes), hipHostMallocMapped | hipHostMallocPortable);
  if (e != hipSuccess) return hip_fail(e, "hipHostMalloc");
  void* dp = nullptr;
  e = hipHostGetDevicePointer(&dp, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return hip_fail(e, "hipHostGetDevicePointer");
  }
  if (dp != p) {
    (void)hipHostFree(p);
    return fail(PSK_E_ARG, "pinned host memory is not mapped at its host address (%p vs %p)", p, dp);
  }
  *ptr = p;
  return PSK_OK;
}

int psk_host_free(void* ptr) {
  g_err[0] = 0;
  if (!ptr) return PSK_OK;
  hipError_t e = hipHostFree(ptr);
  return e == hipSuccess ? PSK_OK : hip_fail(e, "hipHostFree");
}

int psk_keyed_hash(const void* data, int64_t nbytes, uint64_t prefix, int has_prefix, uint64_t* key_out) {
  g_err[0] = 0;
  if (nbytes < 0 || (nbytes && !data) || !key_out) return fail(PSK_E_ARG, "bad hash input (%lld bytes)", (long long)nbytes);
  std::vector<uint8_t> buf(has_prefix ? size_t(nbytes) + 8 : 0);
  *key_out = keyed_digest(static_cast<const uint8_t*>(data), size_t(nbytes), prefix, has_prefix != 0, buf.data());
  return PSK_OK;
}

int64_t psk_page_hash_chain(const void* tokens, int64_t num_tokens, int64_t elem_bytes, int64_t page_size,
                            uint64_t prefix, int has_prefix, uint64_t* keys_out, int64_t keys_capacity) {
  g_err[0] = 0;
  if (num_tokens < 0 || elem_bytes <= 0 || page_size <= 0 || (num_tokens && !tokens))
    return fail(PSK_E_ARG, "bad page-hash geometry (tokens=%lld elem_bytes=%lld page_size=%lld)",
                (long long)num_tokens, (long long)elem_bytes, (long long)page_size);
  const int64_t pages = num_tokens / page_size;
  if (pages > keys_capacity || (pages && !keys_out))
    return fail(PSK_E_WORKSPACE, "%lld page keys do not fit %lld", (long long)pages, (long long)keys_capacity);
  const size_t page_bytes = size_t(page_size) * size_t(elem_bytes);
  std::vector<uint8_t> buf(page_bytes + 8);
  const uint8_t* src = static_cast<const uint8_t*>(tokens);
  uint64_t key = prefix;
  bool chained = has_prefix != 0;
  for (int64_t i = 0; i < pages; ++i, src += page_bytes) {
    key = keyed_digest(src, page_bytes, key, chained, buf.data());
    keys_out[i] = key;
    chained = true;
  }
  return pages;
}

}  // extern "C"
