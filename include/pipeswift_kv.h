/*
 * pipeswift_kv.h -- C ABI of the MI355X (gfx950) paged KV-cache data path.
 *
 * One shared library, libpipeswift_kv.so, built with hipcc for gfx950 from
 * pipeswift_amd/csrc/{pipeswift_kv,paged_attention,mla_fp8_tiles}.hip.  Every
 * entry point takes plain device
 * pointers, element or byte strides and sizes, a dtype code and a HIP stream
 * handle (hipStream_t passed as void*; NULL is the legacy default stream).
 *
 * Conventions shared by every entry point:
 *   - Nothing here allocates device memory or synchronizes the stream, so every
 *     kernel entry point is safe to capture into a HIP graph.
 *   - Return value: PSK_OK (0) on success; a negative PSK_E* code when an
 *     argument violates a precondition (the Python layer raises AssertionError);
 *     a positive hipError_t when the runtime rejects a launch or copy (the
 *     Python layer raises RuntimeError).  psk_last_error() returns a message
 *     for the calling thread's most recent failure.
 *   - Device-side indices (slot_mapping, block tables, block mappings) that fall
 *     outside the cache are skipped by the kernels instead of dereferenced; the
 *     host layer validates them where they live on the host.
 *
 * Reference interfaces each entry replaces (wsjdsg/PipeSwift, Python/Triton):
 *   psk_reshape_and_cache     pipeswift/utils/triton_kernels/reshape_and_cache.py:11-135
 *   psk_concat_and_cache_mla  pipeswift/utils/triton_kernels/reshape_and_cache.py:138-229
 *   psk_swap_blocks           pipeswift/utils/copy_engine.py:429-457 (cuMemcpyBatchAsync)
 *   psk_build_kv_metadata     pipeswift/utils/metadata.py:206-348 (per-token Python loop)
 *   psk_build_next_decode_metadata  pipeswift/utils/metadata.py:351-414 (per-sequence loop)
 *   psk_refresh_graph_metadata      pipeswift/utils/cudagraph.py:75-118 (copy_/fill_ sequence)
 *   psk_page_hash_chain,      pipeswift/engine/block_manager.py:220-227, 678-693
 *   psk_keyed_hash            (xxhash.xxh64 per page; host functions)
 * and build-defined operations that have no reference implementation:
 *   psk_gather_cache          page-table reads done inside attention kernels in the
 *                             reference (pipeswift/llms/layers/attention.py:189-211)
 *   psk_copy_blocks           prefix-cache page copy; the reference remaps instead
 *                             (pipeswift/engine/block_manager.py:841-877)
 *   psk_kv_amax_scale,        per-tensor FP8 scale, and the FP8 append with that
 *   psk_reshape_and_cache_amax  scale; the reference fixes it at 1.0
 *                             (pipeswift/utils/fp8_kv.py:1-3, 75-77)
 *   psk_paged_decode_attention  decode over the FP8 cache; the reference calls
 *                             vLLM's FA3 flash_attn_varlen_func for it
 *                             (pipeswift/llms/layers/attention.py:148-187)
 *   psk_paged_prefill_attention  prefill over the FP8 cache, through the same
 *                             FA3 entry (attention.py:166-184, 577-585)
 *   psk_concat_and_cache_mla_fp8_tiles,  the FP8 MLA entry with per-128-element
 *   psk_gather_mla_fp8_tiles  tile scales that the reference's MLA reader would
 *                             need; it rejects FP8 MLA for lack of it
 *                             (pipeswift/utils/arguments.py:459-467)
 */
#ifndef PIPESWIFT_KV_H
#define PIPESWIFT_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define PSK_DTYPE_F32 0
#define PSK_DTYPE_F16 1
#define PSK_DTYPE_BF16 2
#define PSK_DTYPE_FP8_E4M3FN 3 /* OCP E4M3FN: bias 7, max 448, 0x7F/0xFF NaN */

/* status codes (positive values are hipError_t) */
#define PSK_OK 0
#define PSK_E_ARG (-1)       /* shape, stride, size or pointer precondition */
#define PSK_E_DTYPE (-2)     /* unsupported dtype combination */
#define PSK_E_RANGE (-3)     /* host-visible page index out of range */
#define PSK_E_WORKSPACE (-4) /* workspace too small */

/* swap transports */
#define PSK_SWAP_MEMCPY 0 /* one hipMemcpyAsync per (view, run) on the stream */
#define PSK_SWAP_BLIT 2   /* one copy kernel reading/writing mapped pinned memory */

/* Message for the calling thread's most recent non-zero status. */
const char* psk_last_error(void);

/* ABI version of this library. */
int psk_abi_version(void);

/*
 * Paged KV append for MHA/GQA.  Replaces triton_reshape_and_cache_flash
 * (reshape_and_cache.py:83-135) and its kernel (:11-80).
 *
 * For each token t < num_tokens with s = slot_mapping[t]:
 *   s < 0 (padding, foreign DCP token) or s >= num_blocks*block_size: skipped.
 *   blk = s / block_size, off = s % block_size, for h < num_heads, d < head_size:
 *     key_cache  [blk*kc[0] + off*kc[1] + h*kc[2] + d*kc[3]] = q(key  [t*key_stride   + h*head_size + d], k_scale)
 *     value_cache[blk*vc[0] + off*vc[1] + h*vc[2] + d*vc[3]] = q(value[t*value_stride + h*head_size + d], v_scale)
 * Strides are in elements.  The token's [num_heads, head_size] row is read
 * contiguously from its row start, as the reference does (:43-47, :63-64).
 * in_dtype == cache_dtype: q is the identity (bit copy, any dtype).
 * cache_dtype == FP8_E4M3FN, in_dtype in {BF16, F16, F32}:
 *   q(x, s) = e4m3fn_rne(clamp(float(x) / s, -448, 448)),
 *   s = *scale (device fp32) or 1.0 when the pointer is NULL.  At s == 1.0 this
 *   is the reference's IS_FP8 branch (:66-77).  A NaN quotient stores -448
 *   (0xFE), as the reference's clamp with Triton's minnum/maxnum does (:70-75).
 */
int psk_reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                          const int64_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
                          int64_t head_size, int64_t block_size, int64_t num_blocks,
                          int64_t key_stride, int64_t value_stride, const int64_t* key_cache_strides,
                          const int64_t* value_cache_strides, int in_dtype, int cache_dtype,
                          const float* k_scale, const float* v_scale, void* stream);

/*
 * MLA latent-cache append: replaces triton_reshape_and_cache_flash_diffkv
 * (reshape_and_cache.py:191-229) and its kernel (:138-188).
 *
 * For each token t with a valid slot s (as above) the cache row at
 * kv_cache + blk*cache_block_stride + off*cache_page_stride (elements) receives
 * key_len elements read flat from kv_c + t*kv_c_stride followed by value_len
 * elements read flat from k_pe + t*k_pe_stride (the reference's flat tile_pos
 * addressing, :161-188).  FP8: as psk_reshape_and_cache with one scale.
 */
int psk_concat_and_cache_mla(const void* kv_c, const void* k_pe, void* kv_cache,
                             const int64_t* slot_mapping, int64_t num_tokens, int64_t key_len,
                             int64_t value_len, int64_t kv_c_stride, int64_t k_pe_stride,
                             int64_t block_size, int64_t num_blocks, int64_t cache_block_stride,
                             int64_t cache_page_stride, int in_dtype, int cache_dtype,
                             const float* scale, void* stream);

/*
 * Block gather from a paged cache into contiguous rows (build-defined; vLLM's
 * gather_cache convention).  For sequence b < batch_size and output token
 * t in [cu_seq_lens[b], cu_seq_lens[b+1]) with p = (seq_starts ? seq_starts[b] : 0)
 * + t - cu_seq_lens[b]:
 *   blk = block_table[b*block_table_stride + p / block_size], off = p % block_size
 *   dst[t*dst_row_stride + i] = dq(src[blk*cache_block_stride + off*cache_page_stride + i]),
 *   i < row_len.
 * Rows whose blk is outside [0, num_blocks) are written as zeros; output
 * tokens at or beyond cu_seq_lens[batch_size] are left untouched.
 * src1/dst1 (both NULL or both set) gather a second cache (V) with the same
 * geometry in the same launch.  dq: identity when cache_dtype == out_dtype;
 * FP8_E4M3FN cache to BF16/F16/F32 out: round(float(q) * scale).
 */
int psk_gather_cache(const void* src0, const void* src1, void* dst0, void* dst1,
                     const int32_t* block_table, const int32_t* cu_seq_lens,
                     const int32_t* seq_starts, int64_t batch_size, int64_t block_table_stride,
                     int64_t num_tokens, int64_t row_len, int64_t block_size, int64_t num_blocks,
                     int64_t cache_block_stride, int64_t cache_page_stride, int64_t dst_row_stride,
                     int cache_dtype, int out_dtype, const float* scale, void* stream);

/*
 * Block copy inside a layered cache (build-defined, vLLM's copy_blocks
 * convention).  For every layer l < num_layers and pair i < num_pairs with
 * (s, d) = (block_mapping[2i], block_mapping[2i+1]):
 *   bytes [0, block_bytes) at cache + l*layer_stride + d*block_stride
 *     = bytes at cache + l*layer_stride + s*block_stride        (strides in bytes)
 * Pairs with s or d outside [0, num_blocks) are skipped.  Snapshot semantics
 * hold when destinations are unique and disjoint from sources (the host layer
 * checks this); otherwise overlapping pairs race.  Limits: num_layers <= 65535
 * and num_pairs <= 2^24 (one workgroup per (pair, layer) on a 2-D grid);
 * larger calls return PSK_E_ARG.
 */
int psk_copy_blocks(void* cache, int64_t num_layers, int64_t layer_stride, int64_t block_stride,
                    int64_t block_bytes, int64_t num_blocks, const int64_t* block_mapping,
                    int64_t num_pairs, void* stream);

/*
 * Page transfer between two tiers (device <-> pinned host), the transport under
 * CopyEngine.store/load.  Replaces CopyEngine._copy_blocks (copy_engine.py:429-457).
 *
 * View v has src_bases[v], dst_bases[v] and bytes_per_page[v]; run r moves
 * pages [src_start[r], src_start[r]+run_len[r]) to
 * [dst_start[r], dst_start[r]+run_len[r]) in every view:
 *   dst_bases[v] + dst_start[r]*bpb[v]  <-  src_bases[v] + src_start[r]*bpb[v],
 *   run_len[r]*bpb[v] bytes.
 * All arrays are host memory.  Runs outside [0, src_num_pages) or
 * [0, dst_num_pages) return PSK_E_RANGE before anything is enqueued.
 * PSK_SWAP_BLIT needs `staging`: host memory from psk_host_alloc of at least
 * psk_swap_staging_bytes(num_views, pages) bytes that stays untouched until
 * the enqueued work completes, and optionally `desc_dev`, device memory of the
 * same size: the page tables are then copied there (one async H2D on `stream`)
 * and read by the kernel from HBM instead of over the host link.  The other
 * transports ignore both.  Host-tier pointers must come from psk_host_alloc
 * (mapped pinned memory).
 */
int psk_swap_blocks(int transport, const uint64_t* src_bases, const uint64_t* dst_bases,
                    const uint64_t* bytes_per_page, int64_t num_views, const int64_t* src_start,
                    const int64_t* dst_start, const int64_t* run_len, int64_t num_runs,
                    int64_t src_num_pages, int64_t dst_num_pages, void* staging,
                    int64_t staging_bytes, void* desc_dev, int64_t desc_dev_bytes, void* stream);

/*
 * Host-side run coalescing for a page transfer (replaces CopyEngine._coalesce,
 * copy_engine.py:407-427): pairs (src[i], dst[i]) are ordered by src (stable)
 * and consecutive pairs whose src and dst both advance by one merge into a run.
 * Writes the run starts and lengths (arrays of at least n entries) and returns
 * the number of runs, or a negative status.  Page ids must be non-negative.
 */
int64_t psk_coalesce_runs(const int64_t* src, const int64_t* dst, int64_t n, int64_t* run_src,
                          int64_t* run_dst, int64_t* run_len);

/* Staging bytes PSK_SWAP_BLIT needs for num_views views and num_pages pages. */
int64_t psk_swap_staging_bytes(int64_t num_views, int64_t num_pages);

/*
 * Per-tensor FP8 scale from amax (build-defined; the reference uses 1.0).
 * For tensor j in {0, 1} (x1 may be NULL): amax_j = max |x_j| over `rows` rows
 * of `row_len` elements at element stride row_stride_j, NaN ignored;
 * scale_out[j] = amax_j > 0 ? amax_j / qmax : 1.0f (IEEE fp32 divide);
 * amax_out[j] = amax_j when amax_out is not NULL.  Two launches on `stream`:
 * per-workgroup partial maxima into `workspace` (device memory of
 * psk_kv_amax_workspace_len() uint32 words, no initial contents required),
 * then one workgroup that reduces them.  Calls sharing a workspace must be
 * ordered on one stream.
 */
int psk_kv_amax_scale(const void* x0, const void* x1, int64_t rows, int64_t row_len,
                      int64_t row_stride0, int64_t row_stride1, int dtype, float qmax,
                      float* scale_out, float* amax_out, uint32_t* workspace,
                      int64_t workspace_len, void* stream);

int64_t psk_kv_amax_workspace_len(void);

/*
 * psk_kv_amax_scale without a workspace argument: the partial maxima go to a
 * scratch array inside the library (2 x 1024 uint32 words, 8 KiB per GPU, held
 * until the process ends), so the call allocates nothing and needs no buffer
 * beyond its inputs and outputs.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  Results equal
 * psk_kv_amax_scale's.  Every input size fits (the amax kernel writes at most
 * 1024 partials per tensor).  The scratch needs no initial contents; each GPU
 * has one, shared by every call on that GPU, so calls that overlap on one GPU
 * (different streams, no ordering between them) race.  `stream` must belong
 * to the current device; the first call on a device looks the scratch up.
 */
int psk_kv_amax_scale_noalloc(const void* x0, const void* x1, int64_t rows, int64_t row_len,
                              int64_t row_stride0, int64_t row_stride1, int dtype, float qmax,
                              float* scale_out, float* amax_out, void* stream);

/*
 * The FP8 append with per-tensor scales from this step's own K and V
 * (build-defined; the reference appends with scale 1.0,
 * pipeswift/utils/fp8_kv.py:1-3, 75-77): psk_kv_amax_scale over key and value
 * ([num_tokens, num_heads * head_size] at key_stride / value_stride elements),
 * then psk_reshape_and_cache into an fp8_e4m3fn cache with k_scale =
 * scales_out[0], v_scale = scales_out[1].  Results (cache bytes, scales_out,
 * amax_out) equal those two calls'.  Decode-sized batches take two launches
 * instead of three: the append's waves reduce the partial maxima themselves
 * and the waves of token 0 write the scales.  Other shapes run the three.
 * `workspace` as psk_kv_amax_scale's.
 */
int psk_reshape_and_cache_amax(const void* key, const void* value, void* key_cache,
                               void* value_cache, const int64_t* slot_mapping,
                               int64_t num_tokens, int64_t num_heads, int64_t head_size,
                               int64_t block_size, int64_t num_blocks, int64_t key_stride,
                               int64_t value_stride, const int64_t* kc, const int64_t* vc,
                               int in_dtype, float qmax, float* scales_out, float* amax_out,
                               uint32_t* workspace, int64_t workspace_len, void* stream);

/*
 * Host-side step metadata (replaces the per-token Python loop of
 * prepare_kv_info, pipeswift/utils/metadata.py:206-348).  For sequence i with
 * page ids page_table_ptrs[i][0 .. page_table_lens[i]) (int32, host memory),
 * num_tokens[i] tokens of which offsets[i] are already cached:
 *   page_table_out[i, :]   the page ids, zero-padded to row_width
 *   lens_q_out[i]          num_tokens - offset;  cu_seqlens_q_out prefix sums
 *   lens_kv_out[i]         num_tokens (dcp_deg == 1) or the tokens of the
 *                          rank's share of the prefix (DCP, metadata.py:246-255)
 *   slot_mapping_out       for each new position p:
 *                          page[p / ps] * ps + p % ps (dcp_deg == 1), or with
 *                          DCP the rank-local slot, -1 for foreign tokens
 *                          (metadata.py:282-295)
 * Returns the token count written, or a negative status (a position with no
 * page returns PSK_E_RANGE, where the reference raises IndexError).
 */
int64_t psk_build_kv_metadata(int64_t num_seqs, const uint64_t* page_table_ptrs,
                              const int64_t* page_table_lens, const int64_t* num_tokens,
                              const int64_t* offsets, int64_t page_size, int64_t dcp_deg,
                              int64_t dcp_rank, int64_t dcp_interleave, int is_decode,
                              int64_t row_width, int32_t* page_table_out, int32_t* cu_seqlens_q_out,
                              int32_t* lens_q_out, int32_t* lens_kv_out, int64_t* slot_mapping_out,
                              int64_t slot_capacity);

/*
 * Graph static-metadata refresh (replaces set_graph_kvcacheinfo,
 * pipeswift/utils/cudagraph.py:75-118, a sequence of about ten copy_/fill_/
 * zero_/arange launches per decode step).  One kernel launch on `stream`, no
 * memset node, so it may itself be captured.  Reads the step's device metadata
 * (src_*: page table [bsz, width] at row stride src_page_table_stride,
 * num_slots slots, lens_q/lens_kv [bsz], cu_seqlens_q [bsz + 1]) and writes the
 * static buffers (dst_*: page table [max_bsz, dst_page_table_width] at row
 * stride dst_page_table_stride, slot_mapping [slot_capacity], lens [max_bsz],
 * cu_seqlens_q [max_bsz + 1]):
 *   page_table[r, c]  = src[r, c]              r < bsz, c < width
 *   slot_mapping[k]   = src[k]                 k < num_slots
 *   lens_q/kv[k], cu_seqlens_q[k <= bsz]       copies
 * and, when bsz != cg_bsz (a padded replay; bsz < cg_bsz <= max_bsz):
 *   page_table[r, c]  = 0                      bsz <= r < max_bsz, c < width
 *   slot_mapping[k]   = -1                     num_slots <= k < slot_capacity
 *   lens_q[k] = pad_q_len, lens_kv[k] = 0      bsz <= k < max_bsz
 *   cu_seqlens_q[bsz + j] = cu_seqlens_q[bsz] + j * pad_q_len,  1 <= j <= max_bsz - bsz
 * Elements not named here keep their contents, as in the reference.
 */
int psk_refresh_graph_metadata(const int32_t* src_page_table, int64_t src_page_table_stride,
                                const int64_t* src_slot_mapping, const int32_t* src_lens_q,
                                const int32_t* src_lens_kv, const int32_t* src_cu_seqlens_q, int64_t bsz,
                                int64_t width, int64_t num_slots, int32_t* dst_page_table,
                                int64_t dst_page_table_stride, int64_t dst_page_table_width,
                                int64_t* dst_slot_mapping, int64_t slot_capacity, int32_t* dst_lens_q,
                                int32_t* dst_lens_kv, int32_t* dst_cu_seqlens_q, int64_t max_bsz, int64_t cg_bsz,
                                int32_t pad_q_len, void* stream);

/*
 * Host-side metadata of the next draft decode step (replaces the per-sequence
 * Python loop of derive_kvcache_info_next_decode_step,
 * pipeswift/utils/metadata.py:351-414).  Sequence i has one new token at
 * positions[i] with page ids page_table_ptrs[i][0 .. page_table_lens[i]):
 *   slot_mapping_out[i] = page[pos / ps] * ps + pos % ps, lens_kv_out[i] = lens_kv_prev[i] + 1
 * with DCP (dcp_deg > 1) the rank-local slot when the rank owns pos, else -1
 * with lens_kv unchanged (metadata.py:390-403).  Returns num_seqs, or
 * PSK_E_RANGE when a position has no page (the reference raises IndexError).
 */
int64_t psk_build_next_decode_metadata(int64_t num_seqs, const uint64_t* page_table_ptrs,
                                       const int64_t* page_table_lens, const int64_t* positions,
                                       const int32_t* lens_kv_prev, int64_t page_size, int64_t dcp_deg,
                                       int64_t dcp_rank, int64_t dcp_interleave, int64_t* slot_mapping_out,
                                       int32_t* lens_kv_out);

/*
 * Paged decode attention over an FP8 E4M3FN KV cache (replaces the reader the
 * reference calls through vLLM's FA3 fork, pipeswift/llms/layers/attention.py:
 * 148-187, which takes an FP8 query and per-(sequence, kv head) descales).
 * Decode and speculative decode: sequence b has n_b query tokens, the last n_b
 * positions of the sequence, at rows [c_b, c_b + n_b) of q and out, with
 * c_b = cu_seqlens_q[b] and n_b = cu_seqlens_q[b+1] - c_b (cu_seqlens_q NULL:
 * c_b = b * q_len, n_b = q_len); q_len bounds every n_b and
 * q_len * num_q_heads / num_kv_heads must be at most 16.  For query token
 * r = c_b + i, query head hq = h*G + g (G = num_q_heads / num_kv_heads) and
 * keys j < L_i, where L_i = seq_lens[b] - n_b + 1 + i when causal (FA's
 * bottom-right alignment) and seq_lens[b] otherwise:
 *   q~  = e4m3(q[r,hq] / qd)   (q_dtype FP8: q as is)
 *   s_j = softmax_scale * qd * kd * (q~ . K[j,h])
 *   out[r,hq] = vd * sum_j softmax(s)_j V[j,h],   lse[hq,r] = log sum_j exp(s_j)
 * qd/kd/vd = descale[b * stride_b + h * stride_h] (descale_strides holds the
 * (b, h) strides of q, k, v in that order; a NULL descale is 1.0).
 * q: [total_q, Hq, 128] at element strides (q_tok_stride, q_head_stride).
 * k_cache, v_cache: FP8 [num_blocks, block_size, Hkv, 128]; *_strides are the
 * (block, row, head) strides in bytes, every one and both bases 16-byte aligned.
 * Token j of sequence b is row j % block_size of page
 * block_table[b * block_table_stride + j / block_size]; entries past
 * block_table_width or outside [0, num_blocks) read as zero rows.
 * max_seq_len bounds every seq_lens[b] (block_table_width * block_size does).
 * num_splits > 0: how many workgroups share the longest sequence (flash-decoding
 * split, as FA's num_splits; at most 128 are used).  0: the balanced schedule
 * when the block size is a power of two >= 16 and num_seqs <= 1024 (one
 * workgroup per resident slot, each taking an equal share of the batch's
 * 16-token tiles across sequence boundaries, a sequence start priced as
 * extra tiles), otherwise an automatic split count.
 * out: bf16 or f32 at element strides (out_tok_stride, out_head_stride); lse
 * (fp32, optional) at lse[hq * lse_head_stride + r]; a query token that sees
 * no key (a sequence of length 0) writes zeros and lse = -inf.  Rows of q and
 * out outside every [c_b, c_b + n_b) are not touched.  workspace: device floats, at least
 * psk_paged_decode_workspace_len(); no initial contents needed.  Two launches.
 */
int psk_paged_decode_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride, int q_dtype,
                               const void* k_cache, const void* v_cache, const int64_t* k_strides,
                               const int64_t* v_strides, const int32_t* block_table,
                               int64_t block_table_stride, int64_t block_table_width,
                               const int32_t* seq_lens, int64_t num_seqs, int64_t num_q_heads,
                               int64_t num_kv_heads, int64_t head_size, int64_t block_size,
                               int64_t num_blocks, int64_t max_seq_len, int64_t num_splits,
                               int64_t q_len, const int32_t* cu_seqlens_q, int causal,
                               float softmax_scale,
                               const float* q_descale, const float* k_descale,
                               const float* v_descale, const int64_t* descale_strides, void* out,
                               int64_t out_tok_stride, int64_t out_head_stride, int out_dtype,
                               float* lse, int64_t lse_head_stride, float* workspace,
                               int64_t workspace_len, void* stream);

int64_t psk_paged_decode_workspace_len(int64_t num_seqs, int64_t q_len, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t max_seq_len, int64_t num_splits);

/*
 * Paged prefill attention over an FP8 E4M3FN KV cache: what
 * psk_paged_decode_attention computes (same q~, s_j, out, lse, descales,
 * causal rule, page addressing and zero rows for missing pages), for any
 * number of query tokens per sequence -- the prefill and chunked-prefill steps
 * the reference sends through the same FA3 entry
 * (pipeswift/llms/layers/attention.py:166-184, called for prefill at
 * :577-585).  Sequence b has n_b = min(max_seqlen_q, cu_seqlens_q[b+1] -
 * cu_seqlens_q[b]) query tokens at rows [cu_seqlens_q[b], ...) of q and out
 * (cu_seqlens_q NULL: max_seqlen_q rows each, total_q = num_seqs *
 * max_seqlen_q); total_q is the rows of q and bounds cu_seqlens_q[num_seqs].
 * num_q_heads / num_kv_heads is at most 256.  Each workgroup reads its keys
 * once for 256 / (num_q_heads / num_kv_heads) query tokens of one kv head.
 * out rows (bf16 or f32) need 4-element alignment.  workspace: device int32,
 * at least psk_paged_prefill_workspace_len(num_seqs) words, no initial
 * contents needed.  Two launches.
 */
int psk_paged_prefill_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride, int q_dtype,
                                const void* k_cache, const void* v_cache, const int64_t* k_strides,
                                const int64_t* v_strides, const int32_t* block_table,
                                int64_t block_table_stride, int64_t block_table_width,
                                const int32_t* seq_lens, int64_t num_seqs, int64_t num_q_heads,
                                int64_t num_kv_heads, int64_t head_size, int64_t block_size,
                                int64_t num_blocks, int64_t total_q, int64_t max_seqlen_q,
                                const int32_t* cu_seqlens_q, int causal, float softmax_scale,
                                const float* q_descale, const float* k_descale,
                                const float* v_descale, const int64_t* descale_strides, void* out,
                                int64_t out_tok_stride, int64_t out_head_stride, int out_dtype,
                                float* lse, int64_t lse_head_stride, int32_t* workspace,
                                int64_t workspace_len, void* stream);

int64_t psk_paged_prefill_workspace_len(int64_t num_seqs);

/*
 * FP8 MLA latent entries with one scale per 128-element tile (build-defined;
 * the entry FlashMLA reads for an FP8 latent cache, which the reference lacks:
 * pipeswift/utils/arguments.py:459-467 rejects FP8 for MLA models).  An entry
 * of psk_mla_fp8_tile_entry_bytes(nope_len, rope_len) = nope_len + 4*tiles +
 * 2*rope_len bytes, tiles = nope_len / 128, holds
 *   [0, nope_len)                          q_i = e4m3fn_rne(clamp(x_i / s_{i/128}, -448, 448))
 *   [nope_len, nope_len + 4*tiles)         s_j, float32
 *   [nope_len + 4*tiles, entry bytes)      the rope part, bf16 bit copies
 * with s_j = max(amax_j / 448, 2^-126) (IEEE fp32 division), amax_j = max |x_i|
 * over tile j ignoring NaN; a NaN x_i stores 0x7F|sign.  DeepSeek-V3 (nope 512,
 * rope 64): 656 bytes.  nope_len: a multiple of 128 up to 8192; rope_len: even,
 * at most 512.  psk_mla_fp8_tile_entry_bytes returns a negative status for
 * other sizes.
 *
 * psk_concat_and_cache_mla_fp8_tiles: for each token t with a valid slot s (as
 * psk_reshape_and_cache) the entry at kv_cache + blk*cache_block_stride +
 * off*cache_page_stride (BYTES) is written from kv_c + t*kv_c_stride and
 * k_pe + t*k_pe_stride (elements, bf16 only).  kv_c rows must be 16-byte
 * aligned and entries 4-byte aligned.
 *
 * psk_gather_mla_fp8_tiles: as psk_gather_cache over these entries, writing
 * rows of nope_len + rope_len bf16 or f32 elements at dst + t*dst_row_stride
 * (BYTES, 16-byte aligned): y_i = round(float(q_i) * s_{i/128}) and the rope
 * part converted exactly.  Rows with no valid block are zeros.
 */
int64_t psk_mla_fp8_tile_entry_bytes(int64_t nope_len, int64_t rope_len);
int psk_concat_and_cache_mla_fp8_tiles(const void* kv_c, const void* k_pe, void* kv_cache,
                                       const int64_t* slot_mapping, int64_t num_tokens,
                                       int64_t nope_len, int64_t rope_len, int64_t kv_c_stride,
                                       int64_t k_pe_stride, int64_t block_size, int64_t num_blocks,
                                       int64_t cache_block_stride, int64_t cache_page_stride,
                                       int in_dtype, void* stream);
int psk_gather_mla_fp8_tiles(const void* kv_cache, void* dst, const int32_t* block_table,
                             const int32_t* cu_seq_lens, const int32_t* seq_starts,
                             int64_t batch_size, int64_t block_table_stride, int64_t num_tokens,
                             int64_t nope_len, int64_t rope_len, int64_t block_size,
                             int64_t num_blocks, int64_t cache_block_stride,
                             int64_t cache_page_stride, int64_t dst_row_stride, int out_dtype,
                             void* stream);

/*
 * Pinned, device-mapped host memory for the L2 mirror and swap staging
 * (hipHostMalloc).  Allocation happens at set-up, never on the hot path.
 */
int psk_host_alloc(int64_t bytes, void** ptr);
int psk_host_free(void* ptr);

/*
 * Prefix-cache page keys (replaces BlockManager.compute_hash and the per-page
 * loop of _prompt_page_hashes, pipeswift/engine/block_manager.py:221-227 and
 * :671-689, which call the xxhash package once per page).  Host code.
 *
 * psk_keyed_hash: *key_out = XXH64 (seed 0) of le64(prefix) followed by the
 * `nbytes` bytes at `data`, or of those bytes alone when has_prefix is 0.
 *
 * psk_page_hash_chain: for each full page i of `num_tokens` tokens of
 * `elem_bytes` bytes, keys_out[i] = psk_keyed_hash(page i, keys_out[i-1]),
 * with the caller's (prefix, has_prefix) standing in for keys_out[-1].
 * Returns the number of keys written (num_tokens / page_size), or a negative
 * status (PSK_E_WORKSPACE when keys_capacity is smaller than that).
 */
int psk_keyed_hash(const void* data, int64_t nbytes, uint64_t prefix, int has_prefix,
                   uint64_t* key_out);
int64_t psk_page_hash_chain(const void* tokens, int64_t num_tokens, int64_t elem_bytes,
                            int64_t page_size, uint64_t prefix, int has_prefix,
                            uint64_t* keys_out, int64_t keys_capacity);

#ifdef __cplusplus
}
#endif

#endif /* PIPESWIFT_KV_H */
