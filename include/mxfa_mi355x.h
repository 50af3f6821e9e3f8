/*
 * mxfa_mi355x.h -- C ABI of the MI355X (gfx950) split-KV paged decode library.
 *
 * Library file: mxflashattn_amd/_lib/libmxfa_mi355x.so
 *
 * Every entry point is plain C: raw device pointers, element strides and sizes,
 * an int return code and a hipStream_t passed as void*. Nothing here allocates
 * device memory, synchronises the stream or throws. All launches are
 * asynchronous on the given stream and are safe to record into a HIP graph
 * (no host reads of device data, no memsets).
 *
 * Layouts (elements, not bytes; the last dimension of every tensor must be
 * contiguous and every base pointer 16-byte aligned; an fp8 cache's element is
 * one byte):
 *   q        [B, HQ, HD]                 strides (q_stride_b, q_stride_h, 1)
 *   cache    [num_pages, PS, HKV, HD]    strides (page, token, head, 1)
 *   out      [B, HQ, HD]                 strides (out_stride_b, out_stride_h, 1)
 *   block_table int32 [B, >=ceil(L/PS)]  row stride bt_stride
 *   seqlens  int32 [B]; the attended length of sequence b is seqlens[b] + seqlen_add
 * Query head h reads kv head h / (HQ / HKV).
 * Page ids read from block_table are clamped to [0, num_pages) and lengths to
 * block_table_width * PS, so malformed metadata yields wrong numbers, never an
 * out-of-bounds access.
 *
 * Return codes: MXFA_OK (0) or one of the negative MXFA_E* values below.
 */
#ifndef MXFA_MI355X_H
#define MXFA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXFA_ABI_VERSION 12

/* Return codes. */
#define MXFA_OK 0
#define MXFA_EUNSUPPORTED (-1) /* shape/dtype outside the kernel contract (GQ, HD, dtype, PS) */
#define MXFA_EINVAL (-2)       /* null pointer, non-positive size, misaligned pointer or stride */
#define MXFA_EWORKSPACE (-3)   /* workspace missing or smaller than mxfa_split_decode_workspace_size */
#define MXFA_ELAUNCH (-4)      /* the HIP runtime rejected a kernel launch */
#define MXFA_ESCRATCH (-5)     /* the call needs more than MXFA_SCRATCH_BYTES (no-allocation entry point) */

/* Element types. */
#define MXFA_DTYPE_F16 0
#define MXFA_DTYPE_BF16 1
#define MXFA_DTYPE_FP8_E4M3 2 /* KV caches only (OCP e4m3fn) */

/*
 * num_splits value for the per-sequence kernel: one launch, no workspace.
 * Every workgroup takes one sequence for one kv head; its four waves take
 * every fourth 16-token tile each and merge their partial results in LDS.
 * mxfa_split_heuristic returns it for batches of short sequences (judged by
 * the block table's capacity, block_table_width * page_size), where it skips
 * the tile scan and the second launch. Callers may also pass it themselves.
 * No reference counterpart (the reference always launches partial + combine).
 */
#define MXFA_SPLITS_PER_SEQUENCE (-1)

/* ABI version of the loaded library (MXFA_ABI_VERSION). No reference counterpart. */
int mxfa_abi_version(void);

/* Static text for a return code. No reference counterpart. */
const char *mxfa_strerror(int code);

/*
 * Split count for the launch below, sized for the device's CU count. The
 * work split itself happens on the device: the 16-token tiles of all
 * sequences are laid end to end and cut into num_splits equal ranges (fewer
 * when there are fewer tiles), and every (kv head, range) pair is one wave, so
 * the per-CU load is even for any length mix. When the block table's capacity
 * C = block_table_width * page_size bounds every sequence to a few tiles, it
 * returns MXFA_SPLITS_PER_SEQUENCE instead: page_size >= 16, W = batch *
 * kv_heads * ceil(C / 16) <= 16384, and either head rows of <= 128 bytes with
 * C <= 768 tokens, or 256-byte rows with C <= 384 (or C <= 512 when batch *
 * kv_heads >= 64), and W <= 8192 at head dim 256; never for longer rows, nor
 * when the kernel's 64 KB of LDS cannot hold q_heads / kv_heads columns at this
 * head dim (16 at head dim 256). For mxfa_split_decode_multi_launch pass
 * q_heads * q_len as q_heads (the columns of one launch); the range count
 * does not depend on it. Integer-only, reads no device data. Replaces the Python loop at
 * integrations/vllm/vllm_plugin.py:271-276 (NP doubling until B*HKV*NP >= 2048,
 * c_len = ceil(BTW*PS/NP)).
 */
int mxfa_split_heuristic(int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                         int block_table_width, int num_cus, int *num_splits);

/*
 * Split count for mxfa_split_decode_fp8_launch (same arguments as
 * mxfa_split_heuristic). The launch shape follows the bytes of one head row,
 * so an fp8 cache with head dim HD is sized like a 16-bit cache with HD/2.
 * No reference counterpart (the reference has no fp8 cache).
 */
int mxfa_split_heuristic_fp8(int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                             int block_table_width, int num_cus, int *num_splits);

/*
 * Bytes of caller-owned workspace the split launch needs. Replaces the
 * per-call at::empty of ows/mdws at csrc_native/m1_binding.cpp:94-96. Layout:
 * piece outputs fp32 [HKV, num_splits, 2, GQ, HD], piece base-2 LSEs fp32
 * [HKV, num_splits, 2, GQ] (HKV * GQ = q_heads), tile prefix sums int32
 * [batch + 1]. Its contents between calls do not matter. 0 bytes for
 * MXFA_SPLITS_PER_SEQUENCE (the workspace arguments may then be null and 0).
 */
int mxfa_split_decode_workspace_size(int batch, int q_heads, int head_dim, int num_splits,
                                     size_t *bytes);

/*
 * Split-KV paged decode: out[b, h, :] = softmax(q[b,h]·K_b^T · scale) · V_b over the
 * first seqlens[b] + seqlen_add tokens of sequence b, gathered through block_table.
 * Two launches on `stream`: the split partial kernel (it writes every sequence
 * that lies inside one work range, zero for empty sequences, and the pieces of
 * the others to the workspace), then the LSE combine kernel; with num_splits =
 * MXFA_SPLITS_PER_SEQUENCE one launch of the per-sequence kernel. A sequence of
 * length 0 yields zeros. Calls that share a workspace must not run concurrently.
 *
 * Replaces mxfa_paged_decode_split_launch (csrc_native/m1_kernel.cpp:1206-1211)
 * and its two launches (partial, then split_combine, :985-1001): the same
 * information plus explicit strides, seqlen_add and a sized workspace; the
 * per-split length c_len is gone because ranges are cut on the device.
 * Supported: HD in {64,128,256}, HQ/HKV in 1..16, PS a power of two in
 * [1, 4096], dtype F16/BF16 (q, caches and out share it), batch <= 16000,
 * non-overlapping token rows (cache_stride_token >= HD when PS > 1) and query
 * heads (q_stride_h >= HD). The reference supports HD {64,128} and HQ/HKV
 * {2,4,8} only (integrations/vllm/vllm_plugin.py:220-261 hands the rest back).
 */
int mxfa_split_decode_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                             const void *k_cache, const void *v_cache,
                             int64_t cache_stride_page, int64_t cache_stride_token,
                             int64_t cache_stride_head, const int32_t *block_table,
                             int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                             void *out, int64_t out_stride_b, int64_t out_stride_h,
                             void *workspace, size_t workspace_bytes, float scale, int batch,
                             int q_heads, int kv_heads, int head_dim, int page_size,
                             int block_table_width, int num_pages, int dtype, int num_splits,
                             void *stream);

/*
 * mxfa_split_decode_launch without the workspace arguments, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc). No reference counterpart.
 *
 * The workspace is the library's own device array of MXFA_SCRATCH_BYTES, one
 * per GPU, held until the process ends; calls needing more
 * (mxfa_split_decode_workspace_size > MXFA_SCRATCH_BYTES) return
 * MXFA_ESCRATCH. Nothing in it must start at zero (every byte a call reads was
 * written earlier in that call). Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (different streams) race and
 * give wrong results; serialise them on one stream. Same arguments, kernels
 * and results as mxfa_split_decode_launch otherwise.
 */
#define MXFA_SCRATCH_BYTES ((size_t)8 << 20)
int mxfa_split_decode_noalloc_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void *k_cache, const void *v_cache,
                                     int64_t cache_stride_page, int64_t cache_stride_token,
                                     int64_t cache_stride_head, const int32_t *block_table,
                                     int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                                     void *out, int64_t out_stride_b, int64_t out_stride_h,
                                     float scale, int batch, int q_heads, int kv_heads,
                                     int head_dim, int page_size, int block_table_width,
                                     int num_pages, int dtype, int num_splits, void *stream);

/*
 * Decode with q_len query tokens per sequence (1 <= q_len, q_len * HQ/HKV <=
 * 16), for speculative decoding: q and out are [B, q_len, HQ, HD] with strides
 * (stride_b, stride_t, stride_h, 1). Token t of sequence b sits at position
 * L_b - q_len + t, L_b = seqlens[b] + seqlen_add; here seqlen_add may be
 * negative (>= -2^30; an L_b below 0 counts as 0), so a caller can run the
 * tokens [a, e) of a longer causal query as q_len = e - a tokens with
 * seqlen_add lowered by (its q_len) - e: positions, masks and distances stay
 * those of the whole query. With causal != 0 it attends
 * keys [0, L_b - q_len + t] (bottom-right aligned, as
 * mxflashattn/reference.py:31-35), else all L_b keys; a token with no key gets
 * zeros (the reference's nan_to_num). window_left >= 0 is a sliding window:
 * the token at position i also drops keys before i - window_left
 * (FlashAttention's window_size (window_left, 0) with causal, (window_left,
 * -1) without); -1 means none. sinks, if not null, holds one fp32 logit per
 * query head (HQ values, 4-byte aligned, on the scale of the scaled scores):
 * each output row becomes sum_j e^(s_j) v_j / (sum_j e^(s_j) + e^(sinks[h])),
 * a softmax with one extra zero-valued column (the "s_aux" of vLLM's
 * FlashAttention). softcap > 0 caps every scaled score s to softcap *
 * tanh(s / softcap) before the mask and softmax (FlashAttention's softcap); 0
 * means none. alibi_slopes, if not null, holds one fp32 slope per query head
 * (HQ values, 4-byte aligned): -slope * |p - j| is added to the score of the
 * query at position p and key j, after the cap (FlashAttention's
 * alibi_slopes). The reference has none of these: its guards hand windows and
 * ALiBi to the vendor (integrations/vllm/vllm_plugin.py:220-247), it drops
 * s_aux (:335-339), and its API rejects softcap and ALiBi
 * (mxflashattn/validation.py:56-76). kv_dtype is dtype (16-bit caches) or
 * MXFA_DTYPE_FP8_E4M3 with k_scale/v_scale as in mxfa_split_decode_fp8_launch.
 * Workspace: mxfa_split_decode_workspace_size(batch, q_heads * q_len, ...).
 * Partial and combine run as one call. Other arguments as
 * mxfa_split_decode_launch. The reference's M1 takes q_len = 1 only
 * (csrc_native/m1_binding.cpp:81-88); its API routes longer queries to the
 * vendor, ATen or reference backends (mxflashattn/dispatch.py:89-170).
 */
int mxfa_split_decode_multi_launch(
    const void *q, int64_t q_stride_b, int64_t q_stride_t, int64_t q_stride_h, int q_len,
    int causal, int window_left, const float *sinks, float softcap, const float *alibi_slopes,
    const void *k_cache, const void *v_cache, int64_t cache_stride_page,
    int64_t cache_stride_token, int64_t cache_stride_head, const int32_t *block_table,
    int64_t bt_stride, const int32_t *seqlens, int seqlen_add, void *out, int64_t out_stride_b,
    int64_t out_stride_t, int64_t out_stride_h, void *workspace, size_t workspace_bytes,
    float scale, int batch, int q_heads, int kv_heads, int head_dim, int page_size,
    int block_table_width, int num_pages, int dtype, int kv_dtype, const float *k_scale,
    const float *v_scale, int num_splits, void *stream);

/*
 * Partial stage alone: the first of the two launches of mxfa_split_decode_launch,
 * same arguments. It writes every sequence that lies inside one work range
 * (and zeros for empty sequences) to out, and the normalised output and base-2
 * LSE of every piece of the other sequences, with the tile prefix sums, to the
 * workspace. Followed by mxfa_split_decode_combine_launch on the same stream it
 * is the same computation as mxfa_split_decode_launch; alone it lets a caller
 * time the dominant kernel or schedule the two stages itself. With num_splits
 * = MXFA_SPLITS_PER_SEQUENCE it runs the per-sequence kernel, the whole call.
 * Counterpart of the paged_decode_v3 launch inside launch_split
 * (csrc_native/m1_kernel.cpp:985-999).
 */
int mxfa_split_decode_partial_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void *k_cache, const void *v_cache,
                                     int64_t cache_stride_page, int64_t cache_stride_token,
                                     int64_t cache_stride_head, const int32_t *block_table,
                                     int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                                     void *out, int64_t out_stride_b, int64_t out_stride_h,
                                     void *workspace, size_t workspace_bytes, float scale,
                                     int batch, int q_heads, int kv_heads, int head_dim,
                                     int page_size, int block_table_width, int num_pages,
                                     int dtype, int num_splits, void *stream);

/*
 * Combine stage alone: LSE merge of the pieces of every sequence that crosses
 * a work range end. The workspace must have been filled by
 * mxfa_split_decode_partial_launch with the same batch, heads, head_dim and
 * num_splits, earlier on the same stream; a workspace holding anything else
 * gives wrong numbers (never an out-of-bounds access). With num_splits =
 * MXFA_SPLITS_PER_SEQUENCE there is nothing to merge: it returns MXFA_OK and
 * launches nothing.
 * Counterpart of the split_combine launch (csrc_native/m1_kernel.cpp:1000-1001,
 * kernel :861-888).
 */
int mxfa_split_decode_combine_launch(void *workspace, size_t workspace_bytes, void *out,
                                     int64_t out_stride_b, int64_t out_stride_h, int batch,
                                     int q_heads, int kv_heads, int head_dim, int dtype,
                                     int num_splits, void *stream);

/*
 * Split-KV paged decode over an fp8 KV cache (OCP e4m3fn, one byte per
 * element): out = softmax(q.(k_scale*K)^T * scale) . (v_scale*V). Arguments as
 * mxfa_split_decode_launch, with cache strides in bytes (multiples of 16) and
 * `dtype` naming q and out (F16/BF16); k_scale and v_scale point to one fp32
 * each in device memory (nullptr: 1.0), read by the kernel, so a captured
 * graph sees later updates. K and V are widened exactly to dtype on the
 * device; the scales fold into the score scale and the output normalisation.
 * Uses the same workspace size and combine as the 16-bit launch.
 * No reference counterpart: the reference has no fp8 cache
 * (docs/support-matrix.md:27). For callers with an fp8 vLLM cache
 * (kv_cache_dtype "fp8"/"fp8_e4m3"); num_splits from mxfa_split_heuristic_fp8.
 */
int mxfa_split_decode_fp8_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void *k_cache, const void *v_cache,
                                 int64_t cache_stride_page, int64_t cache_stride_token,
                                 int64_t cache_stride_head, const int32_t *block_table,
                                 int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                                 void *out, int64_t out_stride_b, int64_t out_stride_h,
                                 void *workspace, size_t workspace_bytes, float scale, int batch,
                                 int q_heads, int kv_heads, int head_dim, int page_size,
                                 int block_table_width, int num_pages, int dtype, int num_splits,
                                 const float *k_scale, const float *v_scale, void *stream);

/*
 * Partial stage alone of mxfa_split_decode_fp8_launch (same arguments);
 * followed by mxfa_split_decode_combine_launch it is the same computation.
 * No reference counterpart (see mxfa_split_decode_fp8_launch).
 */
int mxfa_split_decode_fp8_partial_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                         const void *k_cache, const void *v_cache,
                                         int64_t cache_stride_page, int64_t cache_stride_token,
                                         int64_t cache_stride_head, const int32_t *block_table,
                                         int64_t bt_stride, const int32_t *seqlens,
                                         int seqlen_add, void *out, int64_t out_stride_b,
                                         int64_t out_stride_h, void *workspace,
                                         size_t workspace_bytes, float scale, int batch,
                                         int q_heads, int kv_heads, int head_dim, int page_size,
                                         int block_table_width, int num_pages, int dtype,
                                         int num_splits, const float *k_scale,
                                         const float *v_scale, void *stream);

/*
 * Streaming probe (a measurement aid): the split partial kernel's gather with
 * no attention math. Same tile scan, balanced ranges, launch shape and
 * per-tile buffer loads of K and V (q once per piece) as
 * mxfa_split_decode_partial_launch with the same arguments, but each wave
 * only XORs the words it loads; lane l of the wave of (kv head h, range r)
 * writes its XOR to sink[(h * num_splits + r) * 64 + l] (sink_bytes >=
 * kv_heads * num_splits * 256). Ranges r >= the total of 16-token tiles do not
 * exist and are not written; nothing else is. tiles_in_flight: 0 for the decode kernel's own register sets
 * at this head dim, or 2..4 (tiles a wave holds in registers; loads go out
 * tiles_in_flight - 1 tiles ahead). 16-bit caches, head dim 64 or 128, page
 * size >= 16, num_splits > 0. Its time is the ceiling that the decode
 * kernel's access pattern allows on the device.
 *
 * Replaces mxfa_stream_probe (csrc_native/m1_kernel.cpp:1023-1108, bound as
 * mxmmain.stream_probe at csrc_native/m1_binding.cpp:28-35,122-123), which
 * walks each sequence's pages with the decode kernel's row pattern; this one
 * walks the balanced ranges the decode kernel walks.
 */
int mxfa_stream_probe_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                             const void *k_cache, const void *v_cache,
                             int64_t cache_stride_page, int64_t cache_stride_token,
                             int64_t cache_stride_head, const int32_t *block_table,
                             int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                             uint32_t *sink, size_t sink_bytes, int batch, int q_heads,
                             int kv_heads, int head_dim, int page_size, int block_table_width,
                             int num_pages, int dtype, int num_splits, int tiles_in_flight,
                             void *stream);

/*
 * Plain streaming read (a measurement aid; no counterpart in the reference,
 * whose bandwidth probe is the paged one above): reads [buf, buf + bytes)
 * once with 16-byte non-temporal buffer loads and no other work, the read
 * ceiling of the device at a given byte count. `workgroups` workgroups of four
 * waves; each wave reads chunks of `depth` KB (depth 4, 8 or 16: 16-byte loads
 * per lane in flight). layout 0: wave w reads the w-th of 4 * workgroups equal
 * contiguous slices; layout 1: the waves take consecutive chunks in turn.
 * Lane l of wave w writes the XOR of the words it read to sink[64 w + l]
 * (sink_bytes >= workgroups * 1024). buf 16-byte aligned, bytes a positive
 * multiple of 16. Returns MXFA_EINVAL, MXFA_EUNSUPPORTED (depth) or
 * MXFA_EWORKSPACE (sink) before launching anything.
 */
int mxfa_stream_read_launch(const void *buf, uint64_t bytes, int layout, int depth,
                            int workgroups, uint32_t *sink, size_t sink_bytes, void *stream);

/*
 * vLLM-style paged append: for token t with slot = slot_mapping[t] >= 0,
 * cache[slot / PS, slot % PS, kvh, :] = key/value[t, kvh, :]; slot < 0 is skipped.
 * Bit-exact copy. key/value are [num_tokens, HKV, HD] with strides (tok, head, 1).
 * Replaces the vendor reshape_and_cache_flash the reference plugin binds
 * (integrations/vllm/vllm_plugin.py:43-44, do_kv_cache_update :507-511).
 */
int mxfa_reshape_and_cache_launch(const void *key, const void *value,
                                  int64_t kv_stride_token, int64_t kv_stride_head,
                                  void *k_cache, void *v_cache, int64_t cache_stride_page,
                                  int64_t cache_stride_token, int64_t cache_stride_head,
                                  const int64_t *slot_mapping, int num_tokens, int kv_heads,
                                  int head_dim, int page_size, int num_pages, int dtype,
                                  void *stream);

/*
 * vLLM-style paged append into an fp8 cache (kv_cache_dtype "fp8"): as
 * mxfa_reshape_and_cache_launch, but each element becomes
 * e4m3fn_rne(saturate(x / scale, +-448)) with x widened exactly from dtype,
 * the division correctly rounded in fp32, scale = *k_scale for K and *v_scale
 * for V (device pointers, nullptr: 1.0), NaN kept NaN. Cache strides in bytes,
 * multiples of 16; HD a multiple of 16. Counterpart of the vendor
 * reshape_and_cache_flash called with an fp8 kv_cache_dtype and the layer's
 * scales: the reference plugin reuses the vendor's do_kv_cache_update
 * (integrations/vllm/vllm_plugin.py:507-511), and its decode path has no fp8
 * support (docs/support-matrix.md:27). For fp8 vLLM caches.
 */
int mxfa_reshape_and_cache_fp8_launch(const void *key, const void *value,
                                      int64_t kv_stride_token, int64_t kv_stride_head,
                                      void *k_cache, void *v_cache, int64_t cache_stride_page,
                                      int64_t cache_stride_token, int64_t cache_stride_head,
                                      const int64_t *slot_mapping, int num_tokens, int kv_heads,
                                      int head_dim, int page_size, int num_pages, int dtype,
                                      const float *k_scale, const float *v_scale, void *stream);

/*
 * Block-table append used by flash_attn_with_kvcache(k=, v=): token t of
 * sequence b goes to logical position seqlens[b] + t, i.e. page
 * block_table[b, pos / PS], offset pos % PS. seqlens is not modified.
 * k/v are [B, S_new, HKV, HD] with strides (b, tok, head, 1). Bit-exact copy.
 * Replaces the append loop of mxflashattn/reference.py:117-122
 * (csrc/mxmac/paged_kv.cpp:102-109 in the ATen backend).
 */
int mxfa_append_kv_launch(const void *k, const void *v, int64_t kv_stride_b,
                          int64_t kv_stride_token, int64_t kv_stride_head, void *k_cache,
                          void *v_cache, int64_t cache_stride_page, int64_t cache_stride_token,
                          int64_t cache_stride_head, const int32_t *block_table,
                          int64_t bt_stride, const int32_t *seqlens, int batch, int new_tokens,
                          int kv_heads, int head_dim, int page_size, int block_table_width,
                          int num_pages, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFA_MI355X_H */
