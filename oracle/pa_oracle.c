/*
 * pa_oracle.c - CPU restatement of iian's paged-attention path (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never does.
 *
 * Parity status of each function (how it is pinned; tests/test_oracle.py):
 *   pao_f32_to_f16 / pao_f16_to_f32    numpy float16 casts (IEEE RNE), all
 *                                       65536 halves and 2^20 random floats
 *   pao_quantize_row_q8_0 (+ _ref)      bit-exact against ggml's own
 *                                       quantize_row_q8_0 / _ref compiled
 *                                       from the reference tree (oracle/_ref),
 *                                       plus a tie case separating RNE from
 *                                       roundf
 *   pao_dequantize_row_q8_0             ggml's dequantize_row_q8_0 (oracle/_ref)
 *                                       and the closed form q*fp32(d)
 *   pao_set_rows                        closed form: placement by slot, all
 *                                       other rows untouched
 *   pao_paged_attention                 float64 brute-force softmax(qK^T)V
 *                                       with explicit masks, and invariants
 *                                       (block permutation, prefix sharing,
 *                                       thread count, single cell, SWA >= ctx)
 * The reference's paged_attn.cpp itself cannot be built here (it links
 * ggml.c, which needs the CMake-generated ggml-version.h), so the exact fp32
 * bits of paged_attn_impl are restated, not compared.
 */
#include "pa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__F16C__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------ fp16 */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, written from the format
 * definitions.  Restates the conversion of ggml-cpu.c:3480-3499 (F16C,
 * _MM_FROUND_TO_NEAREST_INT); NaNs keep their top payload bits and are
 * quietened as F16C does. */
uint16_t pao_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t) ((ax >> 13) & 0x3ffu);
    }
    const int e = (int) (ax >> 23) - 127;
    if (e >= 16) return sign | 0x7c00u;             /* overflow -> inf */
    if (e >= -14) {                                 /* normal half */
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t h = ((uint32_t) (e + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;  /* may carry into inf */
        return sign | (uint16_t) h;
    }
    if (e < -25) return sign;                       /* below half of the smallest subnormal */
    /* subnormal half: value = m24 * 2^(e-23), unit 2^-24 */
    const uint32_t m24 = (ax & 0x7fffffu) | 0x800000u;
    const int sh = -(e + 1);                        /* 14 .. 24 */
    uint32_t h = m24 >> sh;
    const uint32_t rem = m24 & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return sign | (uint16_t) h;
}

/* binary16 -> binary32, exact (ggml-impl.h:384-405 computes the same value). */
float pao_f16_to_f32(uint16_t hv) {
    const uint32_t sign = ((uint32_t) hv & 0x8000u) << 16;
    const uint32_t ex = (hv >> 10) & 0x1fu;
    const uint32_t m = hv & 0x3ffu;
    if (ex == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
    if (ex == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in binary32 */
        const float v = (float) m * 0x1p-24f;
        return sign ? -v : v;
    }
    return u2f(sign | ((ex + 112u) << 23) | (m << 13));
}

void pao_f32_to_f16_row(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = pao_f32_to_f16(x[i]);
}

void pao_f16_to_f32_row(const uint16_t *x, float *y, int64_t n) {
    int64_t i = 0;
#if defined(__F16C__) && defined(__AVX__)
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(y + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (x + i))));
#endif
    for (; i < n; i++) y[i] = pao_f16_to_f32(x[i]);
}

/* ------------------------------------------------------------------ Q8_0 */

typedef struct { uint16_t d; int8_t qs[PAO_QK8_0]; } q8_0_block;   /* ggml-common.h:251-256 */
_Static_assert(sizeof(q8_0_block) == PAO_Q8_0_BLOCK_BYTES, "block_q8_0 is 34 bytes");

static inline int8_t sat_i8(int32_t v) {   /* packs_epi32 then packs_epi16 saturate */
    if (v > 127) return 127;
    if (v < -128) return -128;
    return (int8_t) v;
}

/* ggml-cpu/arch/x86/quants.c:302-398 (the AVX2 branch the reference engine
 * runs on the MI355X host): per 32 values amax = max|x|, d = amax/127.f,
 * stored as f16(d); id = 127.f/amax (0 when amax == 0); q = RNE(x*id). */
void pao_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    q8_0_block *y = (q8_0_block *) vy;
    const int64_t nb = k / PAO_QK8_0;
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * PAO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < PAO_QK8_0; j++) { const float a = fabsf(xb[j]); amax = a > amax ? a : amax; }
        const float d = amax / 127.f;
        y[b].d = pao_f32_to_f16(d);
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        for (int j = 0; j < PAO_QK8_0; j++) y[b].qs[j] = sat_i8((int32_t) nearbyintf(xb[j] * id));
    }
}

/* ggml-quants.c:276-299: id = 1/d and roundf (ties away from zero). */
void pao_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    q8_0_block *y = (q8_0_block *) vy;
    const int64_t nb = k / PAO_QK8_0;
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * PAO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < PAO_QK8_0; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = pao_f32_to_f16(d);
        for (int j = 0; j < PAO_QK8_0; j++) y[b].qs[j] = (int8_t) roundf(xb[j] * id);
    }
}

/* ggml-quants.c:553-567 */
void pao_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const q8_0_block *x = (const q8_0_block *) vx;
    const int64_t nb = k / PAO_QK8_0;
    for (int64_t b = 0; b < nb; b++) {
        const float d = pao_f16_to_f32(x[b].d);
        for (int j = 0; j < PAO_QK8_0; j++) y[b * PAO_QK8_0 + j] = (float) x[b].qs[j] * d;
    }
}

int64_t pao_row_bytes(int type, int64_t n) {
    switch (type) {
        case PAO_F32: return n * 4;
        case PAO_F16: return n * 2;
        case PAO_Q8_0: return (n / PAO_QK8_0) * PAO_Q8_0_BLOCK_BYTES;
        default: return -1;
    }
}

/* ------------------------------------------------------------- KV write */

/* ggml-cpu/ops.cpp:5221-5289 for an f32 source: for each row i, the index
 * slots[i] must satisfy 0 <= idx < ne1 (GGML_ASSERT :5263) and the row is
 * written with the destination type's from_float (ggml-cpu.c:222-227,
 * 272-273). */
int pao_set_rows(const float *rows, int64_t n_rows, int64_t row_elems,
                 const int64_t *slots, void *pool, int64_t n_cells, int type) {
    const int64_t rb = pao_row_bytes(type, row_elems);
    if (rb < 0 || (type == PAO_Q8_0 && row_elems % PAO_QK8_0)) return -2;
    for (int64_t i = 0; i < n_rows; i++)
        if (slots[i] < 0 || slots[i] >= n_cells) return -1;
    for (int64_t i = 0; i < n_rows; i++) {
        const float *src = rows + i * row_elems;
        char *dst = (char *) pool + slots[i] * rb;
        if (type == PAO_F32) memcpy(dst, src, (size_t) rb);
        else if (type == PAO_F16) pao_f32_to_f16_row(src, (uint16_t *) dst, row_elems);
        else pao_quantize_row_q8_0(src, dst, row_elems);
    }
    return 0;
}

/* ------------------------------------------------------------ attention */

/* Kern<T>::dot of paged_attn.cpp:25-71: two 8-lane FMA accumulators over
 * 16-wide strides, one more 8-wide step, lane-wise a0+a1, then the eight
 * lanes summed left to right; scalar tail after that. */
static inline float dot_f32(const float *q, const float *k, int D) {
    float a0[8] = {0}, a1[8] = {0};
    int i = 0;
    for (; i + 16 <= D; i += 16)
        for (int j = 0; j < 8; j++) {
            a0[j] = fmaf(q[i + j], k[i + j], a0[j]);
            a1[j] = fmaf(q[i + 8 + j], k[i + 8 + j], a1[j]);
        }
    for (; i + 8 <= D; i += 8)
        for (int j = 0; j < 8; j++) a0[j] = fmaf(q[i + j], k[i + j], a0[j]);
    for (int j = 0; j < 8; j++) a0[j] += a1[j];
    float s = a0[0] + a0[1] + a0[2] + a0[3] + a0[4] + a0[5] + a0[6] + a0[7];
    for (; i < D; i++) s = fmaf(q[i], k[i], s);
    return s;
}

/* Kern<T>::axpy of paged_attn.cpp:43-53,77-86: acc += p*v, 8-wide FMA. */
static inline void axpy_f32(float *acc, float p, const float *v, int D) {
    for (int i = 0; i < D; i++) acc[i] = fmaf(p, v[i], acc[i]);
}

typedef struct {
    const float *q;
    const char *k_pool, *v_pool;
    int k_type, v_type;
    const int32_t *bt;
    int32_t max_blocks;
    const int32_t *seq_lens, *seq_idx, *pos;
    int32_t T, S, H, Hkv, D, Dv, bs;
    float scale, softcap;
    int32_t causal, n_swa;
    float *out;
    const int64_t *items;
    int64_t n_items;
    int64_t k_row, v_row;      /* bytes per cell row */
    int32_t max_len;
    int64_t i0, i1;            /* this worker's item range */
} pa_job;

/* Widen one head slice of one cell row to f32 (F16 as in F16C cvtph,
 * Q8_0 via dequantize_row_q8_0, F32 copied). */
static inline const float *head_row(const char *pool, int type, int64_t row_bytes, int64_t cell,
                                    int hk, int d, float *buf) {
    const char *row = pool + cell * row_bytes;
    if (type == PAO_F32) return (const float *) row + (int64_t) hk * d;
    if (type == PAO_F16) { pao_f16_to_f32_row((const uint16_t *) row + (int64_t) hk * d, buf, d); return buf; }
    pao_dequantize_row_q8_0(row + (int64_t) hk * (d / PAO_QK8_0) * PAO_Q8_0_BLOCK_BYTES, buf, d);
    return buf;
}

/* paged_attn_impl<TK,TV> (paged_attn.cpp:90-146) over items [i0, i1). */
static void *pa_worker(void *arg) {
    pa_job *J = (pa_job *) arg;
    float *scores = (float *) malloc(sizeof(float) * (size_t) (J->max_len > 0 ? J->max_len : 1));
    float *acc = (float *) malloc(sizeof(float) * (size_t) J->Dv);
    float *kbuf = (float *) malloc(sizeof(float) * (size_t) J->D);
    float *vbuf = (float *) malloc(sizeof(float) * (size_t) J->Dv);
    const int gqa = J->H / J->Hkv;
    for (int64_t ii = J->i0; ii < J->i1; ii++) {
        const int64_t it = J->items ? J->items[ii] : ii;
        const int64_t t = it / J->H, h = it % J->H, hk = h / gqa;
        const float *qv = J->q + (t * J->H + h) * J->D;
        const int32_t s = J->seq_idx[t];
        const int32_t p1 = J->pos[t];
        const int32_t n_cells = J->seq_lens[s];
        const int32_t *bt = J->bt + (int64_t) s * J->max_blocks;
        /* pass 1: scores and max over the cells this query may attend (:121-130) */
        float mx = -INFINITY;
        for (int32_t c = 0; c < n_cells; c++) {
            const int32_t p0 = c;   /* cell_pos[c] == c (engine.cpp:505) */
            if ((J->causal && p0 > p1) || (J->n_swa > 0 && p1 - p0 >= J->n_swa)) { scores[c] = -INFINITY; continue; }
            const int64_t cell = (int64_t) bt[c / J->bs] * J->bs + c % J->bs;   /* kv_cache.h:135-137 */
            const float *kp = head_row(J->k_pool, J->k_type, J->k_row, cell, (int) hk, J->D, kbuf);
            float sc = dot_f32(qv, kp, J->D) * J->scale;
            if (J->softcap > 0.0f) sc = J->softcap * tanhf(sc / J->softcap);
            scores[c] = sc;
            mx = mx < sc ? sc : mx;
        }
        float *o = J->out + (t * J->H + h) * J->Dv;
        if (mx == -INFINITY) { for (int i = 0; i < J->Dv; i++) o[i] = 0.0f; continue; }   /* :132 */
        /* pass 2: softmax weights and the weighted V sum (:134-144) */
        for (int i = 0; i < J->Dv; i++) acc[i] = 0.0f;
        float sum = 0.0f;
        for (int32_t c = 0; c < n_cells; c++) {
            if (scores[c] == -INFINITY) continue;
            const float p = expf(scores[c] - mx);
            sum += p;
            const int64_t cell = (int64_t) bt[c / J->bs] * J->bs + c % J->bs;
            const float *vp = head_row(J->v_pool, J->v_type, J->v_row, cell, (int) hk, J->Dv, vbuf);
            axpy_f32(acc, p, vp, J->Dv);
        }
        const float inv = 1.0f / sum;
        for (int i = 0; i < J->Dv; i++) o[i] = acc[i] * inv;
    }
    free(scores); free(acc); free(kbuf); free(vbuf);
    return NULL;
}

static int type_ok(int t) { return t == PAO_F32 || t == PAO_F16 || t == PAO_Q8_0; }

int pao_paged_attention(const float *q, const void *k_pool, const void *v_pool,
                        int k_type, int v_type,
                        const int32_t *block_tables, int32_t max_blocks,
                        const int32_t *seq_lens, const int32_t *seq_idx,
                        const int32_t *pos, int32_t T, int32_t S, int32_t H,
                        int32_t Hkv, int32_t D, int32_t Dv, int32_t block_size,
                        float scale, float softcap, int32_t causal, int32_t n_swa,
                        float *out, int32_t n_threads,
                        const int64_t *items, int64_t n_items) {
    if (!q || !k_pool || !v_pool || !block_tables || !seq_lens || !seq_idx || !pos || !out) return -1;
    if (T < 0 || S <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || D <= 0 || Dv <= 0 || block_size <= 0) return -2;
    if (!type_ok(k_type) || !type_ok(v_type)) return -3;
    if ((k_type == PAO_Q8_0 && D % PAO_QK8_0) || (v_type == PAO_Q8_0 && Dv % PAO_QK8_0)) return -3;
    int32_t max_len = 0;
    for (int32_t s = 0; s < S; s++) {
        if (seq_lens[s] < 0 || seq_lens[s] > max_blocks * block_size) return -4;
        if (seq_lens[s] > max_len) max_len = seq_lens[s];
    }
    for (int32_t t = 0; t < T; t++)
        if (seq_idx[t] < 0 || seq_idx[t] >= S) return -5;
    pa_job base;
    memset(&base, 0, sizeof base);
    base.q = q; base.k_pool = (const char *) k_pool; base.v_pool = (const char *) v_pool;
    base.k_type = k_type; base.v_type = v_type; base.bt = block_tables; base.max_blocks = max_blocks;
    base.seq_lens = seq_lens; base.seq_idx = seq_idx; base.pos = pos;
    base.T = T; base.S = S; base.H = H; base.Hkv = Hkv; base.D = D; base.Dv = Dv; base.bs = block_size;
    base.scale = scale; base.softcap = softcap; base.causal = causal; base.n_swa = n_swa;
    base.out = out; base.items = items;
    base.k_row = pao_row_bytes(k_type, (int64_t) Hkv * D);
    base.v_row = pao_row_bytes(v_type, (int64_t) Hkv * Dv);
    base.max_len = max_len;
    const int64_t n = items ? n_items : (int64_t) T * H;
    int nth = n_threads > 0 ? n_threads : 1;
    if (nth > 256) nth = 256;
    /* contiguous chunks per thread, as paged_attn.cpp:103-106 */
    const int64_t per = (n + nth - 1) / nth;
    pa_job jobs[256];
    pthread_t tid[256];
    for (int i = 0; i < nth; i++) {
        jobs[i] = base;
        jobs[i].i0 = (int64_t) i * per < n ? (int64_t) i * per : n;
        jobs[i].i1 = jobs[i].i0 + per < n ? jobs[i].i0 + per : n;
    }
    if (nth == 1) { pa_worker(&jobs[0]); return 0; }
    for (int i = 0; i < nth; i++) pthread_create(&tid[i], NULL, pa_worker, &jobs[i]);
    for (int i = 0; i < nth; i++) pthread_join(tid[i], NULL);
    return 0;
}

/* ---------------------------------------------------------- batch build */

/* The arrays of one engine step that the paged op reads, built the way
 * Engine::step builds its UBatch (src/iian/engine.cpp:491-535) from the
 * scheduler's per-request state, then compressed to block tables:
 *   for request s (batch order), with n_ctx = num_computed[s] + n_new[s]:
 *     cells[i] = cell_of(kv, i), i < n_ctx          (engine.cpp:501-507;
 *                = block_ids[i/bs]*bs + i%bs          kv_cache.h:135-137)
 *     for i in [num_computed, n_ctx): pos = i, seq_idx = s, slot = cell_of(i)
 *                                                    (engine.cpp:508-513)
 *   block_tables[s][b] = block_ids[b] for b < ceil(n_ctx/bs), 0 after;
 *   seq_lens[s] = n_ctx; qsl = exclusive prefix sum of n_new.
 * Request s's block ids are block_ids[block_off[s] .. block_off[s+1]).
 * `cells` (nullable) receives every request's expanded cell list, one after
 * the other; `seq_idx` (nullable) the per-token request index.  Returns the
 * token count T, or -1 when a request's blocks do not cover its context or
 * outnumber max_blocks (the engine's allocate_slots guarantees both,
 * include/iian/kv_cache.h:125-127). */
int64_t pao_build_batch(const int32_t *block_ids, const int32_t *block_off, const int32_t *num_computed,
                        const int32_t *n_new, int32_t S, int32_t block_size, int32_t max_blocks,
                        int32_t *block_tables, int32_t *seq_lens, int32_t *qsl, int32_t *pos, int64_t *slots,
                        int32_t *seq_idx, int64_t *cells) {
    int64_t T = 0, nc = 0;
    qsl[0] = 0;
    for (int32_t s = 0; s < S; s++) {
        const int32_t *ids = block_ids + block_off[s];
        const int32_t nb = block_off[s + 1] - block_off[s];
        const int32_t n_ctx = num_computed[s] + n_new[s];
        if ((int64_t) nb * block_size < n_ctx || nb > max_blocks) return -1;
        for (int32_t i = 0; i < n_ctx && cells; i++)
            cells[nc++] = (int64_t) ids[i / block_size] * block_size + i % block_size;
        for (int32_t i = num_computed[s]; i < n_ctx; i++) {
            pos[T] = i;
            if (seq_idx) seq_idx[T] = s;
            slots[T] = (int64_t) ids[i / block_size] * block_size + i % block_size;
            T++;
        }
        const int32_t used = (n_ctx + block_size - 1) / block_size;
        for (int32_t b = 0; b < max_blocks; b++) block_tables[(int64_t) s * max_blocks + b] = b < used ? ids[b] : 0;
        seq_lens[s] = n_ctx;
        qsl[s + 1] = (int32_t) T;
    }
    return T;
}

/* ------------------------------------------------------------------ RoPE */

/* ggml_rope_yarn_corr_dims (ggml.c:4418-4430): the dims where YaRN's ramp
 * starts and ends. */
static float rope_yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float) M_PI)) / (2 * logf(base));
}

void pao_rope_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow,
                        float dims[2]) {
    const float start = floorf(rope_yarn_corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float end = ceilf(rope_yarn_corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    dims[0] = start > 0 ? start : 0;
    dims[1] = end < n_dims - 1 ? end : (float) (n_dims - 1);
}

/* rope_yarn_ramp (ggml-cpu/ops.cpp:5951-5954). */
static float rope_yarn_ramp(float low, float high, int i0) {
    const float den = high - low > 0.001f ? high - low : 0.001f;
    const float y = (i0 / 2 - low) / den;
    return 1 - (y < 0 ? 0 : (y > 1 ? 1 : y));
}

/* The (cos, sin) cache of one position: ggml_rope_cache_init + rope_yarn
 * (ggml-cpu/ops.cpp:5958-5990): theta starts at the position and is multiplied
 * by theta_scale = powf(freq_base, -2/n_dims) once per pair; each pair's angle
 * is theta / freq_factor, interpolated by freq_scale and, with ext_factor != 0,
 * mixed by the YaRN ramp; the magnitude is attn_factor, times
 * 1 + 0.1 ln(1/freq_scale) with ext_factor != 0.  cos and sin are the
 * correctly rounded fp32 values of the fp32 angle (evaluated in fp64); ggml
 * calls libm cosf / sinf, which differ from those in the last bit on a small
 * fraction of angles (measured in tests/test_oracle.py).  Arithmetic is the
 * C source's, without fused multiply-adds (the oracle is built with
 * -ffp-contract=off).  cache holds n_dims floats: cos, sin per pair. */
void pao_rope_cache(int32_t pos, int n_dims, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                    float attn_factor, float beta_fast, float beta_slow, const float *freq_factors, float *cache) {
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    float corr[2];
    pao_rope_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, corr);
    float theta = (float) pos;
    for (int i0 = 0; i0 < n_dims; i0 += 2) {
        const float ff = freq_factors ? freq_factors[i0 / 2] : 1.0f;
        const float theta_extrap = theta / ff;
        const float theta_interp = freq_scale * theta_extrap;
        float th = theta_interp, mscale = attn_factor;
        if (ext_factor != 0.0f) {
            const float ramp_mix = rope_yarn_ramp(corr[0], corr[1], i0) * ext_factor;
            th = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
        }
        cache[i0 + 0] = (float) cos((double) th) * mscale;
        cache[i0 + 1] = (float) sin((double) th) * mscale;
        theta *= theta_scale;
    }
}

/* ggml_rope_ext forward on f32 rows (ggml_compute_forward_rope_flt,
 * ggml-cpu/ops.cpp:6082-6230; rotate_pairs :6063-6080): each row holds
 * n_heads heads of head_dim values at position pos[row]; the first n_dims
 * values of each head are rotated in pairs (NORMAL, mode 0: (2i, 2i+1);
 * NEOX, mode 2: (i, i + n_dims/2)), y0 = x0 c - x1 s, y1 = x0 s + x1 c, and
 * the rest are copied.  x and y may be the same array.  Returns 0, or -1 for
 * an unsupported mode or n_dims (odd, or above head_dim). */
int pao_rope_rows(const float *x, float *y, int64_t n_rows, int n_heads, int head_dim, const int32_t *pos,
                  int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                  float attn_factor, float beta_fast, float beta_slow, const float *freq_factors) {
    if ((mode != 0 && mode != 2) || n_dims <= 0 || n_dims % 2 || n_dims > head_dim) return -1;
    float *cache = (float *) malloc(sizeof(float) * (size_t) n_dims);
    if (!cache) return -1;
    for (int64_t r = 0; r < n_rows; r++) {
        pao_rope_cache(pos[r], n_dims, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor, beta_fast,
                       beta_slow, freq_factors, cache);
        for (int h = 0; h < n_heads; h++) {
            const float *src = x + (r * n_heads + h) * (int64_t) head_dim;
            float *dst = y + (r * n_heads + h) * (int64_t) head_dim;
            float tmp[1024];
            const float *s = src;
            if (src == dst) { memcpy(tmp, src, sizeof(float) * (size_t) head_dim); s = tmp; }
            for (int i0 = 0; i0 < n_dims; i0 += 2) {
                const int e0 = mode == 0 ? i0 : i0 / 2;
                const int e1 = mode == 0 ? i0 + 1 : i0 / 2 + n_dims / 2;
                const float c = cache[i0], sn = cache[i0 + 1];
                const float x0 = s[e0], x1 = s[e1];
                dst[e0] = x0 * c - x1 * sn;
                dst[e1] = x0 * sn + x1 * c;
            }
            for (int i = n_dims; i < head_dim; i++) dst[i] = s[i];
        }
    }
    free(cache);
    return 0;
}
