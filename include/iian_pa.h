/*
 * iian_pa.h - C ABI of the MI355X paged-attention library (libiian_pa.so).
 *
 * Drop-in for the two operations iian's attention layer performs on the paged
 * KV cache (CocoRoF/iian, paths relative to its source tree):
 *   1. the slot-mapped KV write   ggml_set_rows(cache, rows, slots)
 *                                 (src/iian/graph.cpp:314-322, executed by
 *                                 ggml-cpu/ops.cpp:5221-5289)
 *   2. paged attention            build_paged_attn / paged_attn_op
 *                                 (src/iian/paged_attn.h:16-30,
 *                                 src/iian/paged_attn.cpp:90-169)
 *
 * Conventions
 *   - Every entry point is extern "C", returns an int status (IIAN_PA_OK = 0,
 *     negative on error) and never throws.
 *   - Every pointer argument except `stream` is a device pointer (HBM).  All
 *     launches are asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream).  The caller owns all buffers; the library keeps nothing between
 *     calls except a cached device-property query.
 *   - Type codes are ggml's enum ggml_type values: F32 = 0, F16 = 1, Q8_0 = 8.
 *   - Pool layout is the reference's (src/iian/kv_cache.cpp:156-169): one row
 *     per cell holding all KV heads, K row = Hkv*D elements, V row = Hkv*Dv
 *     elements, rows contiguous; Q8_0 rows are (Hkv*D/32) blocks of 34 bytes
 *     (ggml-common.h:251-256).  Cell of token i of sequence s is
 *     block_tables[s*max_blocks + i/block_size]*block_size + i%block_size
 *     (include/iian/kv_cache.h:135-137).
 */
#ifndef IIAN_PA_H
#define IIAN_PA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    IIAN_PA_OK = 0,
    IIAN_PA_ERR_NULL = -1,         /* a required pointer is NULL */
    IIAN_PA_ERR_ARG = -2,          /* inconsistent sizes / shapes */
    IIAN_PA_ERR_UNSUPPORTED = -3,  /* dtype / head size / ALiBi not supported */
    IIAN_PA_ERR_WORKSPACE = -4,    /* workspace missing or too small */
    IIAN_PA_ERR_HIP = -5,          /* a HIP runtime call failed */
    IIAN_PA_ERR_SCRATCH = -6       /* iian_pa_attention_noalloc: the call needs more than
                                      IIAN_PA_NOALLOC_SCRATCH_BYTES of scratch */
};

/* Size of the library's per-GPU scratch array used by iian_pa_attention_noalloc. */
#define IIAN_PA_NOALLOC_SCRATCH_BYTES ((size_t) 64 << 20)

enum { IIAN_PA_TYPE_F32 = 0, IIAN_PA_TYPE_F16 = 1, IIAN_PA_TYPE_Q8_0 = 8 };

/* Human-readable text of a status code (static storage). */
const char *iian_pa_status_string(int status);

/* Replaces paged_attn_supported (src/iian/paged_attn.cpp:15-18).  Returns 1
 * when iian_pa_attention accepts this combination, else 0.  Accepted: no
 * ALiBi (max_alibi_bias == 0), K and V each F32, F16 or Q8_0 in any pairing
 * (the reference's four F16/F32 pairings, paged_attn.cpp:148-155, widened to
 * Q8_0), and head sizes head_dim (K) and head_dim_v (V, which may differ,
 * paged_attn.cpp:163) from 1 to 1024, multiples of 32 for a Q8_0 pool.
 * The reference accepts any head size (paged_attn.cpp:96-100); sizes above
 * 1024 return 0.
 * Both f16 or both Q8_0 at head size 64, 128 or 256, and both f16 at head
 * size 96, with a power-of-two block size >= 8 run on the MFMA kernels; every
 * other accepted combination runs on the general fp32 kernel (fp32 arithmetic
 * throughout, F32 pools keep full precision). */
int iian_pa_supported(int type_k, int type_v, int head_dim, int head_dim_v, float max_alibi_bias);

/* Replaces ggml_set_rows(cache, rows, slots) on the K or V pool
 * (src/iian/graph.cpp:319-320; CPU semantics ggml-cpu/ops.cpp:5221-5289):
 *   pool row slots[t] <- convert(rows[t]),  t in [0, n_rows)
 * rows: f32 [n_rows][row_elems]; slots: int64 [n_rows]; pool: n_cells rows of
 * `type` (F16: IEEE round-to-nearest-even; Q8_0: ggml's x86 quantiser,
 * ggml-cpu/arch/x86/quants.c:302-398).  Slots must be distinct within a call
 * (ggml.h:1693).  A slot outside [0, n_cells) is not written and sets bit 0 of
 * *err_flag when err_flag is non-NULL (the reference aborts,
 * ggml-cpu/ops.cpp:5263). */
int iian_pa_kv_write(void *stream, const float *rows, int64_t n_rows, int64_t row_elems,
                     const int64_t *slots, void *pool, int64_t n_cells, int type,
                     int32_t *err_flag);

/* The two ggml_set_rows calls of one layer (K pool, then V pool, over the
 * same slots: src/iian/graph.cpp:319-320) as one entry point and, when
 * type_k == type_v, one launch:
 *   k_pool row slots[t] <- convert(k_rows[t]),  v_pool row slots[t] <- convert(v_rows[t])
 * k_rows: f32 [n_rows][k_row_elems]; v_rows: f32 [n_rows][v_row_elems]; both
 * pools hold n_cells rows.  Conversions, slot rules and *err_flag as
 * iian_pa_kv_write. */
int iian_pa_kv_write_kv(void *stream, const float *k_rows, const float *v_rows, int64_t n_rows,
                        int64_t k_row_elems, int64_t v_row_elems, const int64_t *slots,
                        void *k_pool, void *v_pool, int64_t n_cells, int type_k, int type_v,
                        int32_t *err_flag);

/* Bytes of device workspace iian_pa_attention needs for these sizes on the
 * current device (stream-K partial records of the decode rows, or the split
 * records of the general kernel; the size depends on n_seqs, n_head_kv,
 * head_dim_v and the device's compute-unit count only).  Returns 0 on invalid
 * arguments.  No counterpart in the
 * reference, whose CPU op keeps its scratch in thread_local vectors
 * (src/iian/paged_attn.cpp:108-110).  The workspace needs no initialisation and
 * can be reused by later calls on the same stream; concurrent calls (different
 * streams) must not share one. */
size_t iian_pa_workspace_size(int32_t n_tokens, int32_t n_seqs, int32_t n_head, int32_t n_head_kv,
                              int32_t head_dim_v, int32_t max_blocks, int32_t block_size);

/* Replaces build_paged_attn + paged_attn_op (src/iian/paged_attn.h:29-30,
 * src/iian/paged_attn.cpp:90-169).  For every query token t and head h:
 *   out[t][h][:] = sum_c softmax_c(s_c) * V[cell_c][hk][:],
 *   s_c = scale * <q[t][h], K[cell_c][hk]>  (then softcap*tanh(s/softcap)
 *   when softcap > 0), hk = h / (H/Hkv),
 * over the cells c in [0, seq_lens[s]) of the token's sequence s that are not
 * masked: masked when (causal && c > pos[t]) || (n_swa > 0 && pos[t]-c >= n_swa)
 * (paged_attn.cpp:124).  A token with every cell masked gets a zero row
 * (paged_attn.cpp:132).
 *   q               f32 [T][H][D] (contiguous head vectors, paged_attn.cpp:161-162)
 *   k_pool, v_pool  the cell pools of one layer, num_blocks*block_size rows
 *                   (at most 2^32 rows, each under 1 GiB: IIAN_PA_ERR_UNSUPPORTED
 *                   beyond)
 *   block_tables    int32 [S][max_blocks] physical block ids
 *   seq_lens        int32 [S] cells of each sequence, this step's included
 *                   (UBatch::SeqInfo::cells.size(), include/iian/graph.h:33-36)
 *   query_start_loc int32 [S+1] tokens of sequence s are
 *                   [query_start_loc[s], query_start_loc[s+1]) (the
 *                   reference's per-token UBatch::seq_idx, whose tokens are
 *                   contiguous per sequence, engine.cpp:508-513)
 *   pos             int32 [T] UBatch::pos
 *   max_query_len   host int: max tokens of one sequence in this call
 *   out             f32 [T][H][Dv]
 *   workspace       device scratch of at least iian_pa_workspace_size(...) bytes
 *   block_size      any positive size (the reference's is 16, kv_cache.h:27)
 * Bits of *err_flag (when non-NULL; OR-ed in, never cleared):
 *   bit 1  a block id outside [0, num_blocks), or a seq_len beyond the
 *          table's capacity: clamped, never dereferenced out of the pool
 *   bit 2  a sequence has more query tokens than max_query_len: its rows
 *          beyond what the launch covers are not written */
int iian_pa_attention(void *stream, const float *q, const void *k_pool, const void *v_pool,
                      int type_k, int type_v, int32_t num_blocks,
                      const int32_t *block_tables, int32_t max_blocks,
                      const int32_t *seq_lens, const int32_t *query_start_loc,
                      const int32_t *pos, int32_t n_tokens, int32_t n_seqs,
                      int32_t max_query_len, int32_t n_head, int32_t n_head_kv,
                      int32_t head_dim, int32_t head_dim_v, int32_t block_size,
                      float scale, float softcap, int32_t causal, int32_t n_swa,
                      float *out, void *workspace, size_t workspace_bytes,
                      int32_t *err_flag);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  iian_pa_attention without the workspace arguments: the
 * call's scratch (stream-K or split records, segment table, merge counters)
 * lives in a file-scope device array of IIAN_PA_NOALLOC_SCRATCH_BYTES (64 MiB)
 * that the library holds on every GPU it runs on until the process ends.  The
 * call allocates nothing (no hipMalloc, hipFree, stream or event creation; a
 * mixed batch that iian_pa_attention splits over a side stream runs its two
 * kernels in order on `stream` here).  Its first call on a device looks up
 * that device's copy of the array once.  A call needing more scratch than the
 * array holds returns IIAN_PA_ERR_SCRATCH before any launch (every BASELINE
 * configuration fits; the largest uses 34 MB).  Nothing in the array needs
 * clearing between calls: every record is written before it is read within a
 * call, and the merge counters carry a per-call tag.  All calls on one GPU
 * share the array, so calls that overlap on one GPU (different streams, or
 * threads) race: the caller must order them.  Results equal
 * iian_pa_attention's for the same arguments.  Arguments, semantics and
 * *err_flag bits as iian_pa_attention. */
int iian_pa_attention_noalloc(void *stream, const float *q, const void *k_pool, const void *v_pool,
                              int type_k, int type_v, int32_t num_blocks,
                              const int32_t *block_tables, int32_t max_blocks,
                              const int32_t *seq_lens, const int32_t *query_start_loc,
                              const int32_t *pos, int32_t n_tokens, int32_t n_seqs,
                              int32_t max_query_len, int32_t n_head, int32_t n_head_kv,
                              int32_t head_dim, int32_t head_dim_v, int32_t block_size,
                              float scale, float softcap, int32_t causal, int32_t n_swa,
                              float *out, int32_t *err_flag);

/* The layer's KV write and its attention call in one launch, for decode
 * steps: replaces the set_rows of the step's new K and V rows
 * (src/iian/graph.cpp:319-320, iian_pa_kv_write_kv here) followed by the
 * paged attention op (src/iian/graph.cpp:331-336, paged_attn.cpp:90-169,
 * iian_pa_attention here).  New token t's rows k_new[t], v_new[t] (f32
 * [T][n_head_kv*head_dim], 16-byte aligned) are stored, converted to f16 as
 * iian_pa_kv_write converts them, at the cell of its position:
 * block_tables[s][pos[t] / block_size] * block_size + pos[t] % block_size for
 * its sequence s (the slot iian_pa_build_batch computes); then every query
 * attends as iian_pa_attention would after that write.  Pools, outputs and
 * err_flag bits 1 and 2 equal those of the two calls, bit for bit.  Bit 0: a
 * new token whose position is outside [0, seq_lens[s]) or whose block id is
 * outside [0, num_blocks) is not written (the two calls write a slot inside
 * the pool in the second case).  Supported where the call runs the f16
 * decode kernels: f16 pools with head_dim == head_dim_v in {64, 96, 128, 256},
 * a power-of-two block_size of at least 8, max_query_len * n_head / n_head_kv
 * <= 32 (decode and spec-verify steps); anything else returns
 * IIAN_PA_ERR_UNSUPPORTED before any launch, and the caller makes the two
 * calls instead.  Within one call, two new tokens of one sequence at the same
 * position race, as two equal slots of one iian_pa_kv_write call do. */
int iian_pa_write_attention(void *stream, const float *q, const float *k_new, const float *v_new,
                            void *k_pool, void *v_pool, int type_k, int type_v, int32_t num_blocks,
                            const int32_t *block_tables, int32_t max_blocks,
                            const int32_t *seq_lens, const int32_t *query_start_loc,
                            const int32_t *pos, int32_t n_tokens, int32_t n_seqs,
                            int32_t max_query_len, int32_t n_head, int32_t n_head_kv,
                            int32_t head_dim, int32_t head_dim_v, int32_t block_size,
                            float scale, float softcap, int32_t causal, int32_t n_swa,
                            float *out, void *workspace, size_t workspace_bytes,
                            int32_t *err_flag);

/* Builds the arrays iian_pa_attention and iian_pa_kv_write read for one
 * engine step on the device, from the per-request state the scheduler holds,
 * in place of the host loop of Engine::step that expands every request's
 * block table into absolute cells (src/iian/engine.cpp:491-535, cell_of of
 * include/iian/kv_cache.h:135-137): the host uploads sum(blocks) + 3*S
 * integers instead of sum(context) cells.  For request s (batch order):
 *   block_ids[block_off[s] .. block_off[s+1])   KVRequestState::block_ids
 *                                                (kv_cache.h:93-97)
 *   num_computed[s]                              Request::num_computed_tokens
 *   n_new[s]                                     ScheduledRequest::n_new_tokens
 * it writes
 *   seq_lens[s] = num_computed[s] + n_new[s]
 *   query_start_loc[s] = n_new[0] + ... + n_new[s-1], query_start_loc[S] = n_tokens
 *   block_tables[s][b] = the request's b-th block id for the blocks its
 *                        context uses, 0 after them (int32 [S][max_blocks])
 *   pos[t] = num_computed[s] + i and
 *   slots[t] = block_ids[pos/bs]*bs + pos%bs     for its i-th new token t
 *                                                (engine.cpp:508-513)
 * All arrays are device memory.  Bits of *err_flag (when non-NULL):
 *   bit 0  a new token has no block (its slot is -1, which the KV write skips)
 *   bit 1  a block id outside [0, num_blocks)
 *   bit 3  counts inconsistent: negative counts, a request whose blocks do
 *          not cover its context or exceed max_blocks, or new tokens that
 *          do not sum to n_tokens */
int iian_pa_build_batch(void *stream, const int32_t *block_ids, const int32_t *block_off,
                        const int32_t *num_computed, const int32_t *n_new, int32_t n_seqs, int32_t n_tokens,
                        int32_t block_size, int32_t max_blocks, int32_t num_blocks, int32_t *block_tables,
                        int32_t *seq_lens, int32_t *query_start_loc, int32_t *pos, int64_t *slots,
                        int32_t *err_flag);

/* Sliding-window block freeing, the reference's planned "free out-of-window
 * blocks" (docs/ROADMAP.md:33), for a layer with window n_swa > 0: writes to
 * n_free[s] (int32 [S]) the number of leading blocks of sequence s that no
 * query of this step, and none of a later step (whose positions are larger),
 * can see: the blocks that end at or before
 * align_down(min_pos_s - n_swa + 1, 32), where min_pos_s is the smallest
 * position of the sequence's tokens in pos[query_start_loc[s] ..
 * query_start_loc[s+1]).  No attention kernel of this library reads those
 * blocks again (the kernels start a window at that 32-cell boundary), so the
 * block manager may release them from a pool that only sliding-window layers
 * use; their table entries may then hold anything.  When block_tables is
 * non-NULL (int32 [S][max_blocks]), those entries are overwritten with -1.
 * n_swa == 0 (a global layer) frees nothing. */
int iian_pa_swa_free_blocks(void *stream, const int32_t *query_start_loc, const int32_t *pos, int32_t n_seqs,
                            int32_t n_tokens, int32_t n_swa, int32_t block_size, int32_t *n_free,
                            int32_t *block_tables, int32_t max_blocks);

/* Rotary position embedding, as ggml_rope_ext takes it (ggml.h; the
 * arguments build_rope passes, src/iian/graph.cpp:250-253). */
typedef struct {
    int32_t n_dims;              /* rotated values per head (n_rot): even, <= head_dim */
    int32_t mode;                /* 0 = GGML_ROPE_TYPE_NORMAL, 2 = GGML_ROPE_TYPE_NEOX */
    int32_t n_ctx_orig;
    float freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow;
    const float *freq_factors;   /* device, nullable: n_dims/2 divisors (rope_freqs / LongRoPE factors) */
} iian_pa_rope_params;

/* build_rope on K (and q) fused with the layer's two set_rows calls
 * (src/iian/graph.cpp:250-253, 319-320): in one launch, for every token t,
 *   k_pool row slots[t] <- convert(rope(k_rows[t], pos[t])),
 *   v_pool row slots[t] <- convert(v_rows[t]),
 *   q_out[t] <- rope(q_in[t], pos[t])        (when q_in is non-NULL; q_out may equal q_in)
 * k_rows f32 [n_rows][n_head_kv*head_dim], v_rows f32 [n_rows][n_head_kv*head_dim_v],
 * q f32 [n_rows][n_head*head_dim].  rope() is ggml's CPU rope
 * (ggml-cpu/ops.cpp:5951-6230) for modes NORMAL and NEOX: the same chain of
 * fp32 angle products, freq factors, YaRN ramp and magnitude, the pairs
 * rotated with each product rounded; cos and sin are the correctly rounded
 * fp32 values of the fp32 angle, where ggml calls libm cosf / sinf (which can
 * differ in the last bit).  Conversions, slot rules and *err_flag bit 0 as
 * iian_pa_kv_write; q is rotated whatever the slot.  Rows, q and the pools
 * must be 8-byte aligned (IIAN_PA_ERR_ARG otherwise).  Returns
 * IIAN_PA_ERR_UNSUPPORTED for other rope modes, for n_dims above 512, for an
 * odd head size, and for a Q8_0 pool whose head size is not a multiple of 32
 * or is above 512
 * (each head's values are quantised in their own 32-value blocks, as
 * iian_pa_supported requires). */
int iian_pa_rope_kv_write(void *stream, const float *k_rows, const float *v_rows, const float *q_in,
                          float *q_out, const int32_t *pos, const int64_t *slots, int64_t n_rows,
                          int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t head_dim_v,
                          const iian_pa_rope_params *rope, void *k_pool, void *v_pool, int64_t n_cells,
                          int type_k, int type_v, int32_t *err_flag);

/* ---- Engine runtime: the integration point for an engine with its KV cache on the GPU ----
 *
 * Replaces, on the GPU, the step-level work around the paged op: the host
 * UBatch cell expansion of Engine::step (src/iian/engine.cpp:491-535) and the
 * paged branch of GraphContext::build_attn (src/iian/graph.cpp:314-337), which
 * the reference runs on the CPU only (engine.cpp:187-188; its GPU path
 * gathers K/V instead, graph.cpp:487-518).  A runtime owns one step's device
 * buffers (request state, block tables, seq_lens, query_start_loc, pos,
 * slots, attention workspace, error word) and a double-buffered pinned
 * staging area, all allocated by iian_pa_runtime_create for the configured
 * maxima; nothing is allocated afterwards.  One runtime serves one stream at
 * a time. */
typedef struct iian_pa_runtime iian_pa_runtime;

typedef struct {
    int32_t max_seqs;            /* requests per step */
    int32_t max_tokens;          /* new tokens per step */
    int32_t max_blocks_per_seq;  /* block-table row length */
    int32_t max_total_blocks;    /* sum of the step's requests' block counts */
    int32_t n_head, n_head_kv, head_dim, head_dim_v;
    int32_t block_size, num_blocks;
    int32_t type_k, type_v;      /* pool types (iian_pa_supported must accept them) */
} iian_pa_runtime_config;

int iian_pa_runtime_create(const iian_pa_runtime_config *cfg, iian_pa_runtime **out);

/* Waits for every copy and kernel of the device, then frees the runtime (NULL is allowed). */
void iian_pa_runtime_destroy(iian_pa_runtime *rt);

/* Once per engine step, with the scheduler's state of each scheduled request
 * s in batch order (host memory): block_ids[s][0 .. n_blocks[s]) its
 * KVRequestState::block_ids (include/iian/kv_cache.h:93-97), num_computed[s]
 * and n_new[s] its computed and new token counts.  Copies them through pinned
 * memory to the device on `stream` (asynchronously; the caller's arrays may be
 * reused on return) and builds the step's arrays there (iian_pa_build_batch).
 * Returns IIAN_PA_ERR_ARG when a request's blocks do not cover its context or
 * a maximum is exceeded. */
int iian_pa_runtime_begin_step(iian_pa_runtime *rt, void *stream, const int32_t *const *block_ids,
                               const int32_t *n_blocks, const int32_t *num_computed, const int32_t *n_new,
                               int32_t n_seqs);

/* Once per layer of the step: the layer's K/V write into k_pool / v_pool at
 * the step's slots, with RoPE of K and q fused in when rope is non-NULL
 * (iian_pa_rope_kv_write, q rotated into q_rot, which may equal q) or without
 * it (iian_pa_kv_write_kv), then paged attention of q (or q_rot) over the
 * pools into out (iian_pa_attention).  Arrays as those entry points take them. */
int iian_pa_runtime_layer(iian_pa_runtime *rt, void *stream, const float *q, float *q_rot, const float *k_rows,
                          const float *v_rows, const iian_pa_rope_params *rope, void *k_pool, void *v_pool,
                          float scale, float softcap, int32_t causal, int32_t n_swa, float *out);

/* Reads (synchronising `stream`) and clears the runtime's accumulated
 * error word: the bits of iian_pa_build_batch, iian_pa_kv_write and
 * iian_pa_attention. */
int iian_pa_runtime_errors(iian_pa_runtime *rt, void *stream, int32_t *host_err);

/* Dequantises n_rows Q8_0 rows of row_elems values each (pool rows
 * rows_idx[i]) to f32, bit-exactly as ggml's dequantize_row_q8_0
 * (ggml-quants.c:553-567).  Rows outside [0, n_cells) produce zeros.
 * These are the values the reference's dequantised path computes with.  The
 * MFMA attention kernels enter K as exactly these values (int8 q in f16, the
 * block scale d applied in fp32 after the product), but V as f16(q*d): q*d
 * rounded once to f16, as P is (pinned through attention outputs by
 * test_q8_attention_stages_v_as_f16_of_q_times_d).  The reference's own GPU
 * path rounds dequantised Q8_0 K and V to f16 the same way before its flash
 * attention (ggml_cast(get_rows(cache), F16), src/iian/graph.cpp:483-484),
 * so f16(q*d) is what iian computes with on a GPU.  A V value beyond the f16
 * range (|q*d| > 65504, possible only when a block scale exceeds 65504/127 ~
 * 516) becomes +-inf there, and the outputs it reaches are not finite (inf,
 * or NaN where a masked cell's zero weight meets it), where the reference's
 * fp32 value stays finite.  The general kernel enters both K and V as
 * exactly these values. */
int iian_pa_dequant_q8_0(void *stream, const void *pool, int64_t n_cells, const int64_t *rows_idx,
                         int64_t n_rows, int64_t row_elems, float *out);

#ifdef __cplusplus
}
#endif

#endif
