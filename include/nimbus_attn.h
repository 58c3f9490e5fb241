/*
 * nimbus_attn.h - C ABI of the MI355X (gfx950) paged-attention library.
 *
 * libnimbus_attn.so replaces the GPU side of Nimbus's attention hot path:
 * the KV slot write, paged decode attention, causal varlen paged prefill
 * attention (with a verify form for uniform short query runs), the fused
 * residual add + RMSNorm on either side of it, the INT8 weight-only
 * matmul of the quantized projections, and the rotary embedding and SiLU
 * gate of the decoder layer around them. Every entry point
 * takes plain device pointers, element strides
 * (not bytes), sizes, a dtype code and an opaque hipStream_t; none allocates,
 * frees, synchronises or reads device memory on the host, so each call can be
 * recorded into a hipGraph. PyTorch (or any caller) owns every buffer.
 *
 * Return value: 0 on success, a negative NIMBUS_ERR_* for arguments rejected
 * before launch, or a positive hipError_t from the launch itself.
 *
 * Caches are [num_blocks, block_size, num_kv_heads, head_dim] with unit
 * stride in the last dimension (nimbus/cache/kv_cache.py:18-25). The
 * attention kernels are tuned for block_size 16 and head_dim 64 or 128; any
 * other block_size >= 1 and head_dim 1..256 runs a general kernel (correct,
 * not tuned; element loads, so no stride alignment asked and no workspace
 * read) through the same entry points, except the two-pass decode entries
 * and the prefill pieces and stream-K forms, which refuse such shapes with
 * NIMBUS_ERR_UNSUPPORTED. Context lengths and block tables are int32, slot
 * mappings int64 (nimbus/runner.py:77-85).
 */
#ifndef NIMBUS_ATTN_H
#define NIMBUS_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NIMBUS_ATTN_ABI_VERSION 15

/* dtype codes */
#define NIMBUS_FLOAT16 0
#define NIMBUS_BFLOAT16 1

/* error codes (negative: rejected before launch) */
#define NIMBUS_OK 0
#define NIMBUS_ERR_INVALID (-1)     /* inconsistent sizes or null pointers */
#define NIMBUS_ERR_UNSUPPORTED (-2) /* shape/dtype outside what the kernels cover */
#define NIMBUS_ERR_ALIGNMENT (-3)   /* a base or stride breaks 16-byte vector access */
#define NIMBUS_ERR_WORKSPACE (-4)   /* workspace missing or too small */
#define NIMBUS_ERR_SCRATCH (-5)     /* call needs more than nimbus_paged_decode_noalloc's scratch */

/* Version of this ABI (NIMBUS_ATTN_ABI_VERSION). */
int nimbus_attn_abi_version(void);

/* Static text for a return code of any entry point. */
const char* nimbus_attn_error_string(int code);

/*
 * KV slot write. Replaces nimbus/kernels/reference.py:14-23 (write_kv:
 * k_cache.view(-1, KV, D).index_copy_(0, slot_mapping, k), same for v),
 * called on every backend at nimbus/model/attention.py:78.
 *
 * For t < num_tokens: flat slot s = slot_mapping[t] (= block*block_size +
 * offset, nimbus/runner.py:61) receives k[t] in k_cache and v[t] in v_cache,
 * bit for bit. k/v rows: element (t, h, d) at t*stride_token + h*stride_head
 * + d. Caches must be contiguous (the reference views them flat).
 * Slots outside [0, num_slots) are skipped instead of written. Duplicate
 * slots leave one of the writers' rows (which one is unspecified, as with
 * index_copy_).
 */
int nimbus_write_kv(const void* k, const void* v, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                    int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim, int64_t k_stride_token,
                    int64_t k_stride_head, int64_t v_stride_token, int64_t v_stride_head, int64_t num_slots,
                    int32_t dtype, void* stream);

/*
 * Bytes of workspace nimbus_paged_decode needs at this batch, head count,
 * head dim and max_context (a pure function of its arguments): the batch's
 * page prefix sum and room for fp32 (O, m, l) pieces of sequences whose
 * pages are split between waves. The workspace carries nothing from one call
 * to the next and needs no initialisation; calls that run concurrently (on
 * different streams) need different workspaces.
 */
int64_t nimbus_paged_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim,
                                            int64_t max_context);

/*
 * Paged decode attention. Replaces nimbus/kernels/paged_attention.py:101-146
 * (paged_decode_attention with _paged_decode_kernel :25-80 and
 * _merge_partitions_kernel :83-98).
 *
 * out[b, h, :] = softmax(scale * q[b, h] . K_b^T) V_b over the first
 * context_lens[b] tokens of sequence b, read through block_tables[b] from
 * kv head h / (num_heads / num_kv_heads). q/out: element (b, h, d) at
 * b*stride_b + h*stride_h + d. The batch's 16-token pages are split evenly
 * over a fixed number of waves per kv-head group (a split may fall inside a
 * sequence; a second pass merges such sequences' pieces). The launch grid
 * depends only on batch, num_kv_heads, max_context (which must be >= every
 * context length; longer contexts are cut to it) and the device's CU count,
 * so a fixed max_context gives a graph-capturable call. batch <= 4096. Page
 * ids outside [0, num_blocks) read page 0 instead of faulting.
 */
int nimbus_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                        const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                        int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                        int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                        int64_t out_stride_b, int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                        int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, int64_t max_context, float scale, int32_t dtype, void* stream);

/*
 * The two passes of nimbus_paged_decode, launchable on their own (same
 * arguments). nimbus_paged_decode_pages (the work of _paged_decode_kernel,
 * paged_attention.py:25-80) writes the output of every sequence one wave
 * held whole and fp32 pieces of the others; nimbus_paged_decode_merge (the
 * work of _merge_partitions_kernel, paged_attention.py:83-98) combines those
 * pieces into the output. Running pages then merge on one stream equals
 * nimbus_paged_decode.
 */
int nimbus_paged_decode_pages(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                              const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                              int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                              int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                              int64_t out_stride_b, int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                              int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int64_t max_context, float scale, int32_t dtype, void* stream);
int nimbus_paged_decode_merge(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                              const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                              int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                              int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                              int64_t out_stride_b, int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                              int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int64_t max_context, float scale, int32_t dtype, void* stream);

/*
 * Allocation-free paged decode. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments and
 * results as nimbus_paged_decode without the workspace: the kernels use a
 * device array of NIMBUS_NOALLOC_SCRATCH_BYTES inside the library instead,
 * one per device, held until the process ends (its address is looked up
 * once per device, on the first call there). A call whose workspace
 * (nimbus_paged_decode_workspace_bytes) exceeds it returns
 * NIMBUS_ERR_SCRATCH without launching. Every call on a device shares that
 * device's array, so calls that overlap on one device (concurrent streams)
 * race: serialise them. Nothing in the array carries over between calls.
 */
#define NIMBUS_NOALLOC_SCRATCH_BYTES (64LL << 20)
int nimbus_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                                const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                                int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                                int64_t out_stride_b, int64_t out_stride_h, int32_t batch, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int64_t max_context,
                                float scale, int32_t dtype, void* stream);

/*
 * Causal varlen paged prefill attention. Replaces
 * nimbus/kernels/prefill_attention.py:93-119 (paged_prefill_attention and
 * _paged_prefill_kernel :25-78).
 *
 * Sequence i owns query rows [query_start[i], query_start[i+1]) of q; with
 * q_len = that count and ctx = context_lens[i], its query j sits at absolute
 * position ctx - q_len + j and attends to cached tokens 0..ctx - q_len + j
 * (already written by nimbus_write_kv) through block_tables[i].
 * prog_seq/prog_m is the tile table of build_programs
 * (prefill_attention.py:81-90): one entry (sequence, first query offset) per
 * NIMBUS_PREFILL_TILE query positions; num_programs entries. Cache strides
 * must satisfy cache_stride_token <= 2^25 and cache_stride_block < 2^30
 * elements (pages are addressed with 32-bit offsets); others return
 * NIMBUS_ERR_UNSUPPORTED.
 */
#define NIMBUS_PREFILL_TILE 64
int nimbus_paged_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                         const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                         int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                         int64_t bt_stride, int32_t bt_width, const int32_t* query_start,
                         const int32_t* context_lens, const int32_t* prog_seq, const int32_t* prog_m,
                         int32_t num_programs, void* out, int64_t out_stride_t, int64_t out_stride_h,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         int32_t dtype, void* stream);

/*
 * nimbus_paged_prefill with heavy tiles' key ranges cut into pieces, for
 * batches whose tiles alone would leave the chip idle while the heaviest
 * tile walks its keys. pieces: [num_pieces][5] int32 = (sequence, first
 * query offset of a NIMBUS_PREFILL_TILE tile, first key block, end key block
 * (64-key blocks; INT32_MAX = to the causal end), workspace slot or -1 for a
 * whole tile written straight to out). A split tile's pieces write fp32
 * (O, m, l) rows to consecutive slots; merges: [num_merges][4] int32 =
 * (sequence, first query offset, first slot, pieces) combines them into out
 * (o = sum O_i 2^(m_i - M) / sum l_i 2^(m_i - M)). Slots at or past
 * num_slots are never written. Workspace:
 * nimbus_paged_prefill_pieces_workspace_bytes(num_slots, num_heads, head_dim).
 */
int64_t nimbus_paged_prefill_pieces_workspace_bytes(int32_t num_slots, int32_t num_heads, int32_t head_dim);
int nimbus_paged_prefill_pieces(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                                int64_t bt_stride, int32_t bt_width, const int32_t* query_start,
                                const int32_t* context_lens, const int32_t* pieces, int32_t num_pieces,
                                const int32_t* merges, int32_t num_merges, int32_t num_slots, void* workspace,
                                int64_t workspace_bytes, void* out, int64_t out_stride_t, int64_t out_stride_h,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                float scale, int32_t dtype, void* stream);

/*
 * nimbus_paged_prefill with the batch's work balanced over the workgroups
 * the chip holds at once (stream-K), for any batch. Per kv-head group, the
 * 64-key blocks of every unit (NIMBUS_PREFILL_TILE / 2 positions of 4 query
 * heads, or the kernel's 128 rows at other GQA ratios) are laid end to end
 * and cut into num_shares contiguous shares; workgroup (share j, kv-head
 * group g) is grid index j * groups + g, and num_shares * groups must not
 * exceed twice the device's CU count (NIMBUS_ERR_UNSUPPORTED otherwise).
 * share_start [num_shares + 1] and pieces [n][8] int32 are the host's plan:
 * share j walks pieces[share_start[j] .. share_start[j+1]) in order, each
 * (sequence, first query of the unit, first key block, end key block
 * (INT32_MAX: the unit's causal end), slot, fix_lo, fix_hi, 0). slot >= 0:
 * the piece's fp32 (O, m, l) go to share slot `slot` of its kv-head group
 * for a later share to fold in; slot -1: the piece finishes its unit,
 * first folding in the pieces of shares [fix_lo, fix_hi), which must be
 * lower than its own (it waits for each to be written), and writes out.
 * Workspace: nimbus_paged_prefill_stream_workspace_bytes(); its first
 * nimbus_paged_prefill_stream_flag_bytes() (the same for every plan, so
 * calls with different plans may share a workspace) must be zero before the
 * first call (flags, then an error word), and a completed call leaves them
 * zero (the error word aside, which turns nonzero if a wait ever gives up on
 * an inconsistent plan). Calls sharing a workspace must not overlap.
 * Replaces the same reference interface as nimbus_paged_prefill
 * (nimbus/kernels/prefill_attention.py:93-119); the plan stands in for the
 * tile table of build_programs (prefill_attention.py:81-90).
 */
int64_t nimbus_paged_prefill_stream_flag_bytes(int32_t num_shares, int32_t num_heads, int32_t num_kv_heads);
int64_t nimbus_paged_prefill_stream_workspace_bytes(int32_t num_shares, int32_t num_heads, int32_t num_kv_heads,
                                                    int32_t head_dim);
int nimbus_paged_prefill_stream(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                                int64_t bt_stride, int32_t bt_width, const int32_t* query_start,
                                const int32_t* context_lens, const int32_t* share_start, const int32_t* pieces,
                                int32_t num_shares, void* workspace, int64_t workspace_bytes, void* out,
                                int64_t out_stride_t, int64_t out_stride_h, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, float scale, int32_t dtype, void* stream);

/*
 * Bytes of workspace nimbus_paged_verify needs (as for the decode workspace,
 * with queries_per_seq columns per head). -1 for queries_per_seq outside
 * [1, 16].
 */
int64_t nimbus_paged_verify_workspace_bytes(int32_t batch, int32_t queries_per_seq, int32_t num_heads,
                                            int32_t head_dim, int64_t max_context);

/*
 * Speculative-verify attention: causal attention of each sequence's newest
 * queries_per_seq tokens over its paged cache, when every sequence has the
 * same number (1..16) of new tokens. Computes what nimbus_paged_prefill
 * computes for query_start = arange(batch + 1) * queries_per_seq (the
 * verification batch of nimbus/spec/engine.py:84-96, which runs
 * nimbus/kernels/prefill_attention.py:93-119 at q_len = k + 1), with the
 * page-split decode kernels: the queries of a sequence are extra MFMA
 * columns, so each K/V page is read once for all of them.
 *
 * q/out hold batch * queries_per_seq token rows in sequence order: row
 * b * queries_per_seq + j is query j of sequence b, which sits at position
 * context_lens[b] - queries_per_seq + j and sees keys up to it (a query
 * that sees no key, when context_lens[b] < queries_per_seq, gives 0). The
 * _b strides are per token row. Every other argument, the workspace rule
 * (sized by nimbus_paged_verify_workspace_bytes) and the grid rule are
 * nimbus_paged_decode's; queries_per_seq = 1 is nimbus_paged_decode.
 */
int nimbus_paged_verify(int32_t queries_per_seq, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                        const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                        int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                        int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                        int64_t out_stride_b, int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                        int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, int64_t max_context, float scale, int32_t dtype, void* stream);

/*
 * Fused residual add + RMSNorm. Replaces nimbus/kernels/rmsnorm.py:21-59
 * (the Triton _rmsnorm_kernel behind rms_norm and add_rms_norm), with the
 * numerics of nimbus/kernels/reference.py:99-112:
 *   s = x + residual (in the element type; written to residual_out),
 *   out = weight * dtype(s * rsqrt(mean(s^2) + eps)) (mean and scale in fp32).
 * residual == NULL is plain RMSNorm of x (residual_out unused). Rows are
 * [rows, cols] with unit element stride and the given row strides, pointers
 * aligned to their 2-byte elements. Any cols runs, as the Triton kernel's
 * masked block takes any row: the chunked kernel when cols is a multiple of
 * 8 and at most 8192, every pointer 16-byte aligned and every row stride a
 * multiple of 8; otherwise a general kernel (an element per thread, for rows
 * no Llama layer has). residual_out may alias x or residual (an in-place
 * residual update): every element is read before it is written, by the
 * thread that writes it. out must not overlap x, residual or residual_out.
 */
int nimbus_add_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t residual_stride,
                        const void* weight, void* out, int64_t out_stride, void* residual_out,
                        int64_t residual_out_stride, int64_t rows, int32_t cols, float eps, int32_t dtype,
                        void* stream);

/*
 * nimbus_add_rms_norm where x is an INT8 projection's output still in split-K
 * partials: partials [splits][rows][cols] fp32 as
 * nimbus_int8_matmul_packed_partials leaves them and scale [cols] the
 * projection's channel scales. Each x element is formed as the projection's
 * reducing launch forms it (the partials summed in split order, times the
 * scale in fp32, rounded to the element type), so out and residual_out are
 * bit for bit those of nimbus_int8_matmul_packed_plan (same plan) followed by
 * nimbus_add_rms_norm. A residual is required; cols a multiple of 8, at most
 * 8192; every pointer 16-byte aligned, row strides multiples of 8. Has no
 * counterpart call in the reference: it folds the projection's reduction into
 * the norm that reads its output next (nimbus/model/llama.py:115-124, around
 * the o_proj and down_proj of nimbus/quant/int8.py's Int8Linear), one launch
 * instead of two.
 */
int nimbus_add_rms_norm_partials(const float* partials, int32_t splits, const void* scale, const void* residual,
                                 int64_t residual_stride, const void* weight, void* out, int64_t out_stride,
                                 void* residual_out, int64_t residual_out_stride, int64_t rows, int32_t cols,
                                 float eps, int32_t dtype, void* stream);

/*
 * Bytes of workspace nimbus_int8_matmul needs for an [m, k] x [n, k]^T
 * product (0 when it runs without one): a pure function of the shape. The
 * workspace carries nothing between calls; concurrent calls need their own.
 */
int64_t nimbus_int8_matmul_workspace_bytes(int64_t m, int32_t n, int32_t k);

/*
 * INT8 weight-only matmul. Replaces nimbus/kernels/int8_matmul.py:26-64
 * (the Triton _int8_matmul_kernel behind int8_matmul, run by Int8Linear,
 * nimbus/quant/int8.py:32-47):
 *   y[i, j] = dtype(fp32(sum_k x[i, k] * w_q[j, k]) * scale[j])
 * x [m, k] and y [m, n] in dtype with row strides x_stride / y_stride
 * (elements); w_q int8 [n, k] with row stride w_stride (bytes); scale [n]
 * in dtype; x, scale and y aligned to their 2-byte elements. Any shape runs,
 * as the Triton kernel's masked tiles take any shape: the tiled kernel when
 * n is a multiple of 4 and k of 16, x, w_q and y are 16-byte aligned, scale
 * 8-byte aligned, x_stride a multiple of 8, w_stride of 16, y_stride of 4,
 * x and w_q each under 2 GiB and m at most 2^21; otherwise a general kernel
 * (one thread per output, k in order; for shapes no model layer has, not for
 * speed, and it needs no workspace). Either way the summation order over k
 * depends only on the shape and layout, so equal inputs give equal outputs.
 */
int nimbus_int8_matmul(const void* x, int64_t x_stride, const void* w_q, int64_t w_stride, const void* scale,
                       void* y, int64_t y_stride, int64_t m, int32_t n, int32_t k, void* workspace,
                       int64_t workspace_bytes, int32_t dtype, void* stream);

/*
 * The INT8 matmul on weights packed in MFMA tile order. Same y as
 * nimbus_int8_matmul (the Triton kernel it replaces reads w_q [N, K] row by
 * row; Int8Linear packs once, when a layer is quantized, so every call
 * streams the weights in 1 KB contiguous pieces). Packed layout: block
 * (nb, kc) of [ceil(n/16)][ceil(k/64)] is 1024 bytes; bytes 16 l .. 16 l + 15
 * of a block hold row 16 nb + l % 16, columns 64 kc + 16 (l / 16) .. +16,
 * zero padded past n and k. The tiled kernel runs when n is a multiple of
 * 4 and k of 8, x, w_packed and y are 16-byte aligned, scale 8-byte aligned,
 * x_stride a multiple of 8 and y_stride of 4 (with nimbus_int8_matmul's size
 * limits); any other call runs the general kernel on the packed layout. The
 * workspace rule is nimbus_int8_matmul's, sized by
 * nimbus_int8_matmul_packed_workspace_bytes (0 for shapes the tiled kernel
 * does not take).
 */
int64_t nimbus_int8_packed_weight_bytes(int32_t n, int32_t k);
int nimbus_int8_pack_weight(const void* w_q, int64_t w_stride, int32_t n, int32_t k, void* out, void* stream);
int64_t nimbus_int8_matmul_packed_workspace_bytes(int64_t m, int32_t n, int32_t k);
int nimbus_int8_matmul_packed(const void* x, int64_t x_stride, const void* w_packed, const void* scale, void* y,
                              int64_t y_stride, int64_t m, int32_t n, int32_t k, void* workspace,
                              int64_t workspace_bytes, int32_t dtype, void* stream);

/*
 * nimbus_int8_matmul_packed with an explicit launch plan, for a caller that
 * tunes per shape (as the reference's triton.autotune does per M bucket,
 * N and K): bm tokens per workgroup tile (16, 32, 64 or 128), ks k slices per
 * workgroup (1, 2, 4 or 8, with ks * bm <= 128), splits of K (1..16) and
 * rows_per_wave 16-row blocks per wave (1 or 2). Any valid plan gives y to
 * fp32 summation order; the workspace is
 * nimbus_int8_matmul_packed_plan_workspace_bytes (-1 for an invalid plan,
 * and for a shape the tiled kernel does not take). A plan runs the tiled
 * kernel only: a call it cannot take returns an error instead of falling
 * back.
 */
int64_t nimbus_int8_matmul_packed_plan_workspace_bytes(int64_t m, int32_t n, int32_t k, int32_t bm, int32_t ks,
                                                       int32_t splits, int32_t rows_per_wave);
int nimbus_int8_matmul_packed_plan(const void* x, int64_t x_stride, const void* w_packed, const void* scale, void* y,
                                   int64_t y_stride, int64_t m, int32_t n, int32_t k, int32_t bm, int32_t ks,
                                   int32_t splits, int32_t rows_per_wave, void* workspace, int64_t workspace_bytes,
                                   int32_t dtype, void* stream);

/*
 * The MLP's gate_up projection and SiLU gate in one launch. Replaces
 * MLP.forward's F.silu(gate) * up over Int8Linear's output
 * (nimbus/model/llama.py:100-103, nimbus/quant/int8.py:43-47): w_packed holds
 * gate_up_proj's n = 2 * intermediate rows (gate rows first), and y [m, n/2]
 * receives what nimbus_silu_mul would make of the [m, n] output of
 * nimbus_int8_matmul_packed_plan under the same plan (bm, ks, one split,
 * rows_per_wave), bit for bit, without that output being written. n a multiple
 * of 32, k of 8; one split of K: bm (16, 32, 64 or 128; 0 picks from m with
 * ks = 1 and one row block per wave), ks (1, 2 or 4, ks * bm <= 128) and
 * rows_per_wave (1 or 2) as for nimbus_int8_matmul_packed_plan. The tiled
 * kernel's alignment and size rules apply (an error otherwise, no other
 * path); y must not overlap x. No workspace.
 */
int nimbus_int8_matmul_packed_silu(const void* x, int64_t x_stride, const void* w_packed, const void* scale, void* y,
                                   int64_t y_stride, int64_t m, int32_t n, int32_t k, int32_t bm, int32_t ks,
                                   int32_t rows_per_wave, int32_t dtype, void* stream);

/*
 * The first half of nimbus_int8_matmul_packed_plan for a plan that splits K
 * (splits >= 2 once the plan is made; NIMBUS_ERR_UNSUPPORTED otherwise): the
 * per-split fp32 sums land in workspace as [splits][m][n]
 * (nimbus_int8_matmul_packed_plan_workspace_bytes() bytes) and no reducing
 * launch follows, for a consumer that folds them in
 * (nimbus_add_rms_norm_partials). Arguments as for
 * nimbus_int8_matmul_packed_plan, less scale and y. Replaces the same
 * reference interface (Int8Linear.forward, nimbus/quant/int8.py:43-47),
 * whose output the next call completes.
 */
int nimbus_int8_matmul_packed_partials(const void* x, int64_t x_stride, const void* w_packed, int64_t m, int32_t n,
                                       int32_t k, int32_t bm, int32_t ks, int32_t splits, int32_t rows_per_wave,
                                       void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream);

/*
 * Rotary position embedding, in place. Replaces Rotary.forward
 * (nimbus/model/llama.py:37-57) on the q and k heads of the fused qkv
 * projection: token t (row stride x_stride elements) holds num_heads heads
 * of head_dim; each head's pairs (i, i + head_dim/2) rotate by the
 * positions[t] row of the fp32 cos / sin tables (row stride table_stride),
 * with every multiply and the add rounded to dtype as the reference's ops
 * are. Tokens whose position is outside [0, max_position) are left as is.
 * head_dim a multiple of 16; x 16-byte aligned, x_stride a multiple of 8;
 * the tables 16-byte aligned with table_stride a multiple of 4.
 */
int nimbus_rope(void* x, int64_t x_stride, int64_t num_tokens, int32_t num_heads, int32_t head_dim,
                const int64_t* positions, const float* cos_table, const float* sin_table, int64_t table_stride,
                int32_t max_position, int32_t dtype, void* stream);

/*
 * Rotary embedding and KV slot write in one launch: exactly nimbus_rope(qkv,
 * qkv_stride, num_tokens, num_heads + num_kv_heads, head_dim, ...) followed
 * by nimbus_write_kv of the k and v heads of the same rows, bit for bit.
 * Replaces the rotary of Attention.forward (nimbus/model/llama.py:88-98)
 * and the write_kv call that AttentionBackend.forward makes first
 * (nimbus/model/attention.py:78). Row t of qkv (row stride qkv_stride
 * elements) holds num_heads q heads, then num_kv_heads k heads, then
 * num_kv_heads v heads, head_dim elements each; the q and k heads are
 * rotated in place, and the rotated k heads and the v heads go to flat
 * slot slot_mapping[t] of the contiguous caches [num_slots, num_kv_heads,
 * head_dim] (slots outside [0, num_slots) skipped, as nimbus_write_kv).
 * Same alignment rules as nimbus_rope, plus 16-byte aligned caches.
 */
int nimbus_rope_write_kv(void* qkv, int64_t qkv_stride, int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                         int32_t head_dim, const int64_t* positions, const float* cos_table, const float* sin_table,
                         int64_t table_stride, int32_t max_position, void* k_cache, void* v_cache,
                         const int64_t* slot_mapping, int64_t num_slots, int32_t dtype, void* stream);

/*
 * SiLU-gated product of the MLP. Replaces F.silu(gate) * up
 * (nimbus/model/llama.py:100-103): row r of x holds [gate | up] (2 * cols
 * elements); out[r] = dtype(dtype(silu(gate)) * up). cols a multiple of 8;
 * x and out 16-byte aligned, strides multiples of 8.
 */
int nimbus_silu_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride, int64_t rows, int32_t cols,
                    int32_t dtype, void* stream);

/*
 * One step of the on-device greedy chain. Replaces the loop body of
 * DecodeGraphs.greedy_chain (nimbus/cuda_graph.py:104-115): for each row r
 * < rows, tok = argmax(logits[r, :vocab]) (first index among equal maxima)
 * becomes input_ids[r]; for rows with active[r] != 0 it is also recorded at
 * tokens[r, context_lens[r] - ctx_start[r]] (when that is < max_steps), and
 * positions[r], context_lens[r] advance by one and slots[r] becomes the
 * cache slot of the new position through block_tables[r] (scratch_slot past
 * the table's width). Inactive rows (padding) only take the token.
 */
int nimbus_greedy_step(const float* logits, int64_t logits_stride, int32_t rows, int32_t vocab, int64_t* input_ids,
                       int64_t* positions, int32_t* context_lens, int64_t* slots, const int32_t* block_tables,
                       int64_t bt_stride, int32_t bt_width, int32_t block_size, const int32_t* active,
                       const int32_t* ctx_start, int64_t* tokens, int32_t max_steps, int64_t scratch_slot,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NIMBUS_ATTN_H */
