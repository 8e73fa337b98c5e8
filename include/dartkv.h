/*
 * dartkv.h — C ABI of the MI355X-native DartKV compressed-KV path.
 *
 * libdartkv_hip.so exports these functions.  Every pointer is a device pointer
 * unless stated otherwise.  Every call enqueues work on the given HIP stream
 * (a hipStream_t passed as void*, NULL = default stream), returns immediately,
 * and returns DKV_OK (0) or an error code.  On error, dkv_last_error() returns a
 * thread-local message.  Nothing here allocates device memory: callers pass
 * outputs and workspace.
 *
 * Element types (the *_dtype arguments) use DKV_DTYPE_*.  Sources, outputs,
 * caches and queries may be float64, float32, float16 or bfloat16 (the page
 * kernels of dkv_decode_attention take bf16 / fp16 caches; everything else
 * takes all four).  As in the reference, quantization runs in the source
 * dtype: a float64 source in IEEE double with eps 1e-6, its float64 scale and
 * minimum converted to a 16-bit metadata dtype through float32, as torch does.
 *
 * Layouts are the reference's tensor layouts (reference src/dart/quantization.py,
 * src/dart/mixed.py), so a reference-side binding can hand over the storage
 * of its QuantizedTensor / MixedQuantizedKey fields unchanged.
 */
#ifndef DARTKV_H
#define DARTKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DKV_DTYPE_F32 0
#define DKV_DTYPE_F16 1
#define DKV_DTYPE_BF16 2
#define DKV_DTYPE_F64 3

#define DKV_OK 0
#define DKV_ERR_INVALID 1     /* bad shape / argument (Python: ValueError)     */
#define DKV_ERR_UNSUPPORTED 2 /* valid but not implemented here (ValueError)   */
#define DKV_ERR_DTYPE 3       /* bad element type (Python: TypeError)          */
#define DKV_ERR_HIP 4         /* HIP runtime failure (Python: RuntimeError)     */

#define DKV_KEY_DENSE 0
#define DKV_KEY_UNIFORM 1
#define DKV_KEY_MIXED 2
#define DKV_VALUE_DENSE 0
#define DKV_VALUE_UNIFORM 1

#define DKV_SELECT_MAGNITUDE 0
#define DKV_SELECT_VARIANCE 1
#define DKV_SELECT_GIVEN 2 /* caller supplies per-head indices ("random" strategy) */

/* Thread-local description of the last error on this thread. */
const char* dkv_last_error(void);

/* ABI version (13); bumps when a struct or an entry point below changes. */
int dkv_abi_version(void);

/*
 * Uniform group quantization of `rows` rows of `n` elements each, groups of
 * `group` consecutive elements, last group padded by repeating the row's last
 * element.  Element (r, i) of the source is at src[r * row_stride + i * elem_stride].
 *
 * Outputs (contiguous): values[rows][packed_bytes] with element i of a row at
 * byte i / (8/bits), bits [(i % (8/bits)) * bits, ...) (LSB first);
 * scale[rows][groups], zero[rows][groups] in meta_dtype.
 *
 * Replaces reference src/dart/quantization.py:134-204 (`quantize`, after its
 * movedim to the last axis) and :213-223 (`quantize_axis`); the cache calls it
 * for value pages (src/dart/cache.py:505-512).
 */
int dkv_quantize_rows(const void* src, int src_dtype, int64_t rows, int64_t n,
                      int64_t row_stride, int64_t elem_stride, int bits, int64_t group,
                      uint8_t* values, void* scale, void* zero, int meta_dtype, void* stream);

/*
 * dkv_quantize_rows over `blocks` blocks of `block_rows` rows each, the form a
 * token slice of a [B, H, T, D] tensor takes: row r = blk * block_rows + i
 * (0 <= i < block_rows) starts at src[blk * block_stride + i * row_stride] and
 * its elements are contiguous.  Outputs are laid out as for dkv_quantize_rows
 * with rows = blocks * block_rows, so the result equals dkv_quantize_rows on
 * the contiguous copy of the slice without making that copy.
 *
 * Replaces the same reference code as dkv_quantize_rows: the cache quantizes
 * value pages cut out of the appended tensor along tokens
 * (src/dart/cache.py:505-512, src/dart/quantization.py:134-204).
 */
int dkv_quantize_row_blocks(const void* src, int src_dtype, int64_t blocks, int64_t block_stride,
                            int64_t block_rows, int64_t n, int64_t row_stride, int bits, int64_t group,
                            uint8_t* values, void* scale, void* zero, int meta_dtype, void* stream);

/*
 * Value rows for dkv_quantize_key_pages to quantize in the same call, with the
 * meaning of dkv_quantize_row_blocks's arguments: `blocks` blocks of
 * `block_rows` rows of `n` contiguous elements, row r = blk * block_rows + i at
 * src[blk * block_stride + i * row_stride]; outputs laid out as for
 * dkv_quantize_rows.
 */
typedef struct dkv_value_rows_args {
  const void* src;
  int64_t src_dtype;
  int64_t blocks, block_stride, block_rows, n, row_stride;
  int64_t bits, group;
  uint8_t* values;
  void* scale;
  void* zero;
  int64_t meta_dtype;
  /* Optional (NULL: no check): a uint32 the device can write (device memory,
   * or pinned host memory, read after a stream synchronization without a
   * copy) set to 1 when a group holds a NaN or an infinity (the reference
   * raises ValueError for such inputs, src/dart/quantization.py:159-160);
   * never cleared by the library. */
  uint32_t* nonfinite;
  /* Output placement: source row blk * block_rows + i goes to output row
   * blk * out_block_rows + out_row0 + i (out_block_rows 0: block_rows, the
   * contiguous layout), so a caller can quantize new token rows straight into
   * a [B][H][capacity][...] store at token offset out_row0. */
  int64_t out_block_rows, out_row0;
} dkv_value_rows_args;

/*
 * dkv_quantize_row_blocks described by a dkv_value_rows_args, with its
 * optional non-finite flag: the form the cache uses for value pages that are
 * quantized without keys (reference src/dart/cache.py:457-470 and :505-512,
 * quantize at src/dart/quantization.py:134-204).
 */
int dkv_quantize_value_rows(const dkv_value_rows_args* args, void* stream);

/*
 * Key quantization along tokens for `n_pages` pages of `page_tokens` tokens.
 * Source keys are [B, H, T, D]; page p covers tokens
 * [p * page_tokens, (p + 1) * page_tokens) of `src`, element (b, h, t, d) at
 * src[b*sb + h*sh + t*st + d*sd].
 *
 * key_mode DKV_KEY_MIXED (Dart promotion, reference src/dart/mixed.py:166-244,
 * channel choice :119-163): per page, fields laid out as the reference's
 *   low   [B][H][D][G][nb]  uint8, nb = ceil(group/4)
 *   high  [B][H][K][G][nb]  uint8 (upper 2 bits of promoted channels, top-k order)
 *   idx   [B][H][K]         int32
 *   scale [B][H][D][G], zero [B][H][D][G] in meta_dtype
 * with G = ceil(page_tokens / group) and K = `promoted`.  `selection` picks the
 * channel score (DKV_SELECT_*); DKV_SELECT_GIVEN reads given_idx[H][K].
 *
 * key_mode DKV_KEY_UNIFORM (reference src/dart/quantization.py:213-223 with
 * axis=-2, as src/dart/cache.py:497-502 calls it):
 *   low   [B][H][D][pk]     uint8 codes of the padded token axis, pk = ceil(G*group / (8/bits))
 *   scale [B][H][D][G], zero [B][H][D][G]
 * (high and idx unused).
 *
 * Page p's fields start at field + p * field_page_stride (strides in bytes).
 * Replaces reference src/dart/cache.py:481-503 (`_quantize_key_pages`).
 */
struct dkv_copy_block; /* defined with dkv_copy_token_blocks below */

typedef struct dkv_key_pages_args {
  const void* src;
  int64_t src_dtype;
  int64_t B, H, D, page_tokens, n_pages;
  int64_t sb, sh, st, sd; /* element strides of the source */
  int64_t key_mode, bits, group, promoted, selection;
  const int32_t* given_idx;
  int64_t meta_dtype;
  uint8_t* low;
  int64_t low_page_stride;
  uint8_t* high;
  int64_t high_page_stride;
  int32_t* idx;
  int64_t idx_page_stride;
  void* scale;
  int64_t scale_page_stride;
  void* zero;
  int64_t zero_page_stride;
  /* Optional (NULL: keys only): the value rows of the same tokens, quantized
   * by this call too.  The reference quantizes a page's keys and its values
   * one after the other (src/dart/cache.py:472-479); given both, the library
   * runs the value kernel alongside the key path's serial channel selection. */
  const dkv_value_rows_args* values;
  /* Optional (NULL: no check): a uint32 the device can write (as in
   * dkv_value_rows_args) set to 1 when a key group holds a NaN or an
   * infinity (reference src/dart/mixed.py:187-188 and
   * src/dart/quantization.py:159-160 raise ValueError); never cleared. */
  uint32_t* nonfinite;
  /* Optional (n_copies 0: none): up to DKV_COPY_MAX_BLOCKS dense token-row
   * copies, with the meaning dkv_copy_token_blocks gives them, made by this
   * call too.  An append keeps its sink tokens and its held tail dense next
   * to the pages it quantizes (reference src/dart/cache.py:183-185 and
   * :417-418, :451-467); given here, the library runs them inside a quantize
   * launch where one has room for them. */
  const struct dkv_copy_block* copies;
  int64_t n_copies;
} dkv_key_pages_args;

int dkv_quantize_key_pages(const dkv_key_pages_args* args, void* stream);

/*
 * Copy the token rows of up to DKV_COPY_MAX_BLOCKS dense blocks in one
 * launch: block j sets dst[b][h][t] = src[b][h][t] (row_bytes bytes) for
 * b < B, h < H, t < T; the strides are in bytes, and a block's source and
 * destination must not overlap.  Blocks of zero rows are skipped.  This is
 * how an append keeps its dense tokens: reference src/dart/cache.py:183-185
 * (the sink tokens' clone) and :417-418, :451-467 (the pending tail's clone).
 */
#define DKV_COPY_MAX_BLOCKS 8

typedef struct dkv_copy_block {
  const void* src;
  void* dst;
  int64_t B, H, T, row_bytes;
  int64_t src_sb, src_sh, src_st;
  int64_t dst_sb, dst_sh, dst_st;
} dkv_copy_block;

int dkv_copy_token_blocks(const dkv_copy_block* blocks, int64_t n_blocks, void* stream);

/*
 * Dequantize `rows` rows produced by dkv_quantize_rows (same layout) into
 * out[r * out_row_stride + i] (i < n) in out_dtype, with the reference's
 * rounding chain: out = to_out(meta(meta(code * scale) + zero)).
 * Replaces reference src/dart/quantization.py:96-109 and the uniform kernels of
 * src/dart/triton_ops.py:32-110.
 */
int dkv_dequantize_rows(const uint8_t* values, const void* scale, const void* zero, int meta_dtype,
                        int64_t rows, int64_t n, int bits, int64_t group, void* out, int out_dtype,
                        int64_t out_row_stride, void* stream);

/*
 * Dequantize mixed keys (layout of dkv_quantize_key_pages, one page of
 * `tokens` tokens) to out[B][H][tokens][D] in out_dtype.
 * Replaces reference src/dart/mixed.py:72-94 and src/dart/triton_ops.py:113-201.
 */
int dkv_dequantize_mixed(const uint8_t* low, const uint8_t* high, const int32_t* idx, const void* scale,
                         const void* zero, int meta_dtype, int64_t B, int64_t H, int64_t D, int64_t tokens,
                         int64_t group, int64_t promoted, void* out, int out_dtype, void* stream);

/*
 * One cache segment (a page, a dense sink piece, the dense pending tail) as
 * the decode kernel sees it.  Field addresses are device addresses; *_bh are
 * strides, in elements of that field, between consecutive (batch, kv-head)
 * blocks.  Inside a block the layouts are those of dkv_quantize_key_pages /
 * dkv_quantize_rows, and a dense block is [tokens][D] with row stride D.
 *   key[0]: dense values | uniform codes | mixed low codes
 *   key[1]: mixed high codes      key[2]: mixed channel indices (int32)
 *   key[3]: scale                 key[4]: zero
 *   value[0]: dense values | codes   value[1]: scale   value[2]: zero
 */
typedef struct dkv_segment {
  int32_t tokens;
  int32_t key_kind;   /* DKV_KEY_*   */
  int32_t value_kind; /* DKV_VALUE_* */
  int32_t key_bits;
  int32_t key_group;
  int32_t promoted;
  int32_t value_bits;
  int32_t value_group;
  uint64_t key[5];
  int64_t key_bh[5];
  uint64_t value[3];
  int64_t value_bh[3];
} dkv_segment;

/*
 * Single-token GQA decode attention over a packed cache: query [B][Hq][D]
 * (element (b,h,d) at query[b*q_sb + h*q_sh + d]) attends to every token of
 * segments[0..n_segments) (device array, in sequence order) and, when
 * tail.tokens > 0, to `tail` (passed by value, last in sequence).  Query head h
 * uses KV head h / (Hq/Hkv).  Logits are (q . k) * scale in fp32 with an online
 * softmax; K and V are dequantized with the reference's rounding chain.
 *
 * Work is split over contiguous segment ranges per (batch, kv head); partial
 * (max, sum, acc[D]) go to `workspace` (dkv_decode_workspace_bytes bytes for
 * n_splits + fast_splits records) and a merge pass writes out[b][h][d]
 * (out_sb, out_sh strides, q dtype) and, if out_f32 != NULL, the fp32 result
 * before the final cast to out_f32[(b*Hq + h)*D + d].
 *
 * Fast page path: when fast_count > 0, descriptor entries
 * [fast_first, fast_first + fast_count) must all be full 128-token pages with
 * head_dim 128, Dart keys with fast_promoted promoted channels (a multiple of
 * 16, at most 64, one key group per page), 2-bit values in groups of
 * fast_value_group channels (a multiple of 16 dividing 128), fp16 metadata and a
 * bf16 or fp16 cache, every field 16-byte aligned, and Hq / Hkv of 1, 2, 4
 * or 8; the caller guarantees this (except the head ratio, which is checked).
 * Those pages are processed by the MFMA page kernel over `fast_splits` splits;
 * the other entries and the tail by the general kernel over `n_splits` splits.
 * With fast_promoted == 0 the run is instead uniform pages: keys quantized
 * with fast_key_bits bits along the tokens (one key group per page), values
 * with fast_value_bits bits along the channels in groups of fast_value_group
 * (2, 4 or 8 bits each), split over half pages (fast_splits at most
 * 2 * fast_count), also with Hq / Hkv of 1, 2, 4 or 8.  For Dart pages
 * fast_key_bits and fast_value_bits are 0 or 2.
 *
 * Dense rest: when rest_dense_tokens > 0 the caller guarantees that every entry
 * outside the fast range and the tail are dense segments in the cache dtype
 * (bf16 or fp16) with 16-byte aligned rows and at most rest_dense_tokens
 * tokens each; then one wave per 32-token chunk handles them (head_dim 128, at
 * most 8 query heads per KV head, n_splits = number of those segments *
 * ceil(rest_dense_tokens / 32)).
 *
 * Checked guarantees: when segments_host is not NULL it holds the same
 * n_segments descriptors in host memory, and every entry of the fast range and,
 * with rest_dense_tokens > 0, every other entry is checked against the rules
 * above (DKV_ERR_INVALID naming the entry); the tail is always checked.
 * Without a host copy the caller guarantees them, and a non-page segment the
 * dense kernel cannot read makes the result NaN instead of wrong.
 *
 * Query range: the page kernels compute with fp16 operands; each split scales
 * its query heads by a power of two that brings the largest |q| into
 * [2^14, 2^15) and takes the inverse power into the logit scale (exact), so any
 * finite query works, and queries in fp16's normal range give the same bits as
 * without the scaling.
 *
 * Timing: fast_events[0] / [1], when not NULL, are hipEvent_t handles recorded
 * on `stream` right before and right after the page kernel's launch.
 *
 * Replayable launches: when tail_tokens_dev is not NULL, the kernels read the
 * tail's token count from that device int64 when they run, clamped to
 * [0, tail.tokens]; tail.tokens then gives the tail's capacity (and sizes the
 * splits).  A caller that captures these launches in a graph and appends to
 * the tail on the device between replays keeps the count there.
 *
 * Replaces reference src/dart/fused_attention.py:654-771
 * (`fused_dart_attention`, one query token) and, for one query token,
 * src/dart/attention.py:32-87 (`streamed_dart_attention`).
 */
typedef struct dkv_decode_args {
  const void* query;
  int64_t q_dtype, q_sb, q_sh;
  void* out;
  int64_t out_sb, out_sh;
  float* out_f32;
  const dkv_segment* segments;
  int64_t n_segments;
  dkv_segment tail;
  int64_t B, Hq, Hkv, D;
  int64_t cache_dtype, meta_dtype;
  double scale;
  int64_t n_splits;
  void* workspace;
  int64_t workspace_bytes;
  int64_t fast_first, fast_count, fast_promoted, fast_value_group, fast_splits;
  int64_t rest_dense_tokens;
  void* fast_events[2];
  const int64_t* tail_tokens_dev;
  int64_t fast_key_bits, fast_value_bits;
  const dkv_segment* segments_host;
} dkv_decode_args;

/*
 * Decode-step preparation for the Qwen3 adapter, one new token per sequence:
 * qkv[b] holds the projected query heads, key heads and value heads of
 * sequence b (Hq + 2 Hkv rows of D = 128 elements, row stride qkv_sb elements,
 * cache dtype bf16 or fp16).  Query and key heads get RMSNorm (fp32 x *
 * rsqrt(mean(x^2) + eps), rounded, times q_weight / k_weight[D], rounded) and
 * the rotary embedding (x*cos + rotate_half(x)*sin, each product and the sum
 * rounded; cos, sin [D] for this token's position).  Queries go to
 * q_out[B][Hq][D]; keys and values to tail_key / tail_value[B][Hkv][cap][D] at
 * token index *tail_pos (a device int64, read when the kernel runs; positions
 * outside [0, cap) write nothing).  *tail_pos itself is not changed.
 *
 * Replaces, for one query token, the Transformers Qwen3 q_norm / k_norm and
 * apply_rotary_pos_emb calls of reference src/dart/integrations/qwen3.py:48-53
 * and the append of the new key/value in src/dart/integrations/huggingface.py:68.
 */
typedef struct dkv_decode_prep_args {
  const void* qkv;
  int64_t qkv_sb;
  const void* q_weight;
  const void* k_weight;
  double eps;
  const void* cos;
  const void* sin;
  void* q_out;
  void* tail_key;
  void* tail_value;
  const int64_t* tail_pos;
  int64_t B, Hq, Hkv, D, cap, dtype;
} dkv_decode_prep_args;

int dkv_decode_prep(const dkv_decode_prep_args* args, void* stream);

int64_t dkv_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t n_splits);

int dkv_decode_attention(const dkv_decode_args* args, void* stream);

/*
 * dkv_decode_attention without a caller workspace and without any device
 * allocation: the split records go to a static device array of
 * dkv_decode_scratch_bytes() bytes (32 MiB) that the library holds on each
 * GPU it runs on until the process ends.  args->workspace and
 * args->workspace_bytes are ignored; every other argument means what it means
 * for dkv_decode_attention.  A call whose records
 * (dkv_decode_workspace_bytes of its splits) exceed the scratch returns
 * DKV_ERR_INVALID.  Calls that overlap on one GPU (several streams or host
 * threads) share the array and race; callers serialize them.
 *
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).
 */
int dkv_decode_attention_noalloc(const dkv_decode_args* args, void* stream);
int64_t dkv_decode_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* DARTKV_H */
