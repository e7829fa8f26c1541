/*
 * pa_oracle.h - CPU restatement of iian's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (iian_amd/, include/) may
 * link, import or call this code.  It is the checker that the HIP kernels are
 * compared against: used by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, and nowhere else.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the CocoRoF/iian source tree).
 *
 * Type codes are ggml's (ggml.h enum ggml_type): F32 = 0, F16 = 1, Q8_0 = 8.
 */
#ifndef PA_ORACLE_H
#define PA_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { PAO_F32 = 0, PAO_F16 = 1, PAO_Q8_0 = 8 };
#define PAO_QK8_0 32
#define PAO_Q8_0_BLOCK_BYTES 34

/* fp32 -> fp16, IEEE round-to-nearest-even (the F16C _mm256_cvtps_ph path of
 * ggml-cpu.c:3480-3499; scalar twin ggml-impl.h:407-431). */
uint16_t pao_f32_to_f16(float f);
/* fp16 -> fp32, exact widening (ggml-impl.h:384-405). */
float pao_f16_to_f32(uint16_t h);
void pao_f32_to_f16_row(const float *x, uint16_t *y, int64_t n);
void pao_f16_to_f32_row(const uint16_t *x, float *y, int64_t n);

/* Q8_0 quantiser actually used by the reference engine on x86 hosts
 * (ggml-cpu/arch/x86/quants.c:302-398): d = amax/127, id = 127/amax,
 * q = round-half-even(x*id), saturating to int8.  k % 32 == 0. */
void pao_quantize_row_q8_0(const float *x, void *y, int64_t k);
/* ggml's scalar reference quantiser (ggml-quants.c:276-299): id = 1/d,
 * q = roundf(x*id) (ties away from zero).  Kept only to document and test the
 * difference from the x86 variant; the KV write follows the x86 variant. */
void pao_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);
/* ggml-quants.c:553-567: y = q * fp32(d), exact in fp32. */
void pao_dequantize_row_q8_0(const void *x, float *y, int64_t k);

/* Bytes of one pool row of `n` elements of `type` (ggml_row_size). */
int64_t pao_row_bytes(int type, int64_t n);

/* Slot-mapped KV write: ggml_set_rows(cache, rows, slots) as emitted by
 * build_attn (graph.cpp:314-322) and executed by
 * ggml_compute_forward_set_rows_impl (ggml-cpu/ops.cpp:5221-5289):
 * pool row slots[t] <- from_float(rows[t]), rows are `row_elems` f32 values.
 * Returns 0, or -1 when a slot is outside [0, n_cells) (the GGML_ASSERT of
 * ops.cpp:5263), or -2 for an unsupported type. */
int pao_set_rows(const float *rows, int64_t n_rows, int64_t row_elems,
                 const int64_t *slots, void *pool, int64_t n_cells, int type);

/*
 * Paged attention: paged_attn_impl<TK,TV> (src/iian/paged_attn.cpp:90-146)
 * for every (token, head) item, with the UBatch of include/iian/graph.h:22-38
 * given in compressed form:
 *   seq_idx[t], pos[t]              UBatch::seq_idx / UBatch::pos
 *   block_tables[s*max_blocks + b]  KVRequestState::block_ids, so that
 *                                   cells[i] = bt[i/bs]*bs + i%bs and
 *                                   cell_pos[i] = i (engine.cpp:501-507,
 *                                   kv_cache.h:135-137)
 *   seq_lens[s]                     seq.cells.size()
 * q is [T][H][D] f32, out is [T][H][Dv] f32; pools hold Hkv*D (K) and Hkv*Dv
 * (V) elements per cell row in k_type / v_type (F32, F16 or Q8_0; Q8_0 is
 * dequantised to f32 and then run through the F32 kernel, which is the only
 * way the reference CPU kernel can consume it, paged_attn.cpp:15-18).
 * n_threads > 1 splits the items into contiguous chunks exactly as
 * paged_attn.cpp:103-106 does; the result does not depend on it.
 * `items` (nullable) restricts the computation to the listed t*H+h items;
 * other output rows are left untouched.
 * Returns 0 or a negative code for invalid arguments.
 */
int pao_paged_attention(const float *q, const void *k_pool, const void *v_pool,
                        int k_type, int v_type,
                        const int32_t *block_tables, int32_t max_blocks,
                        const int32_t *seq_lens, const int32_t *seq_idx,
                        const int32_t *pos, int32_t T, int32_t S, int32_t H,
                        int32_t Hkv, int32_t D, int32_t Dv, int32_t block_size,
                        float scale, float softcap, int32_t causal, int32_t n_swa,
                        float *out, int32_t n_threads,
                        const int64_t *items, int64_t n_items);

/* The arrays of one engine step the paged op reads (block tables, seq_lens,
 * query_start_loc, pos, slots), built as Engine::step builds its UBatch
 * (src/iian/engine.cpp:491-535) from per-request block ids, computed-token
 * counts and new-token counts, then compressed to block tables (padded with
 * 0).  `seq_idx` and `cells` (the expanded per-request cell lists) are
 * optional outputs.  Returns the token count, or -1 when a request's blocks do
 * not cover its context or exceed max_blocks. */
int64_t pao_build_batch(const int32_t *block_ids, const int32_t *block_off, const int32_t *num_computed,
                        const int32_t *n_new, int32_t S, int32_t block_size, int32_t max_blocks,
                        int32_t *block_tables, int32_t *seq_lens, int32_t *qsl, int32_t *pos, int64_t *slots,
                        int32_t *seq_idx, int64_t *cells);

/* RoPE as ggml_rope_ext computes it on the CPU (ggml-cpu/ops.cpp:5951-6230,
 * ggml.c:4418-4430), modes NORMAL (0) and NEOX (2); see pa_oracle.c for the
 * cos/sin evaluation.  pao_rope_cache writes the n_dims (cos, sin) values of
 * one position; pao_rope_rows rotates rows of n_heads heads (x may equal y);
 * pao_rope_corr_dims is ggml_rope_yarn_corr_dims. */
void pao_rope_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow,
                        float dims[2]);
void pao_rope_cache(int32_t pos, int n_dims, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                    float attn_factor, float beta_fast, float beta_slow, const float *freq_factors, float *cache);
int pao_rope_rows(const float *x, float *y, int64_t n_rows, int n_heads, int head_dim, const int32_t *pos,
                  int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                  float attn_factor, float beta_fast, float beta_slow, const float *freq_factors);

#ifdef __cplusplus
}
#endif

#endif
