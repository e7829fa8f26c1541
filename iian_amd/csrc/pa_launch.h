// pa_launch.h - internal launchers shared between the kernel files and the C ABI layer.
#pragma once

#include "pa_common.h"

namespace iian_pa {

// Everything the general fp32 kernel (pa_general.hip) reads, by value.
struct GenParams {
    const float *q;             // [T][H][D]
    const char *k_pool;         // cell rows of Hkv*D elements of the K type
    const char *v_pool;         // cell rows of Hkv*Dv elements of the V type
    const int32_t *bt;          // [S][max_blocks]
    const int32_t *seq_lens;    // [S]
    const int32_t *qsl;         // [S+1]
    const int32_t *pos;         // [T]
    float *out;                 // [T][H][Dv]
    float *part_o;              // split records: [T*H][n_split][Dv]
    float *part_ml;             // [T*H][n_split] of (m in log2 units, l)
    int32_t *err;               // nullable error word
    int64_t k_row, v_row;       // bytes per pool row
    int32_t max_blocks, num_blocks, block_size;
    int32_t T, S, H, Hkv, gqa, D, Dv;
    int32_t max_q;              // the caller's max_query_len
    int32_t rows_per_block;     // query rows per workgroup: 4 or 16 (general_rows_per_block)
    int32_t n_rb;               // row blocks launched per (sequence, kv head)
    int32_t n_split;            // KV ranges per row block (1 .. 64)
    int32_t tile_cells;         // TC: 32, 16 or 8
    float scale, softcap;
    int32_t causal, n_swa;
};

// Waves per segment workgroup of the f16 segment decode kernel
// (pa_decode_seg_kernel, p.seg_waves), by head size, and the most tiles per
// wave a sliding-window call may give it.
constexpr int kSegWavesD64 = 16;
constexpr int kSegWavesD128 = 8;
constexpr int kSegWavesD256 = 4;
constexpr int kSegSwaTilesPerWave = 16;

// Decode / spec-verify kernel (sequences with n_q*gqa <= p.decode_rows) plus the stream-K merge.
hipError_t launch_decode(const AttnParams &p, int head_dim, int kv_type, hipStream_t stream);
// The Q8_0-pool variant of launch_decode (pa_decode_q8.hip).
hipError_t launch_decode_q8(const AttnParams &p, int head_dim, hipStream_t stream);
// Log-sum-exp merge of the decode kernels' stream-K partial records.
hipError_t launch_merge(const AttnParams &p, int head_dim, hipStream_t stream);
// MFMA prefill kernel (sequences with n_q*gqa > p.decode_rows); grid covers max_query_len*gqa rows.
// Q8_0 pools at head size 64 and 128, and both pool types at 256 (f16 pools at
// 64, 96 and 128 take launch_mixed_f16).
hipError_t launch_prefill(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream);
// A mixed batch over an f16 pool at head size 64, 96 or 128 in one launch: prefill
// workgroups plus the decode rows' stream-K workers, which merge their split
// segments themselves.
hipError_t launch_mixed_f16(const AttnParams &p, int head_dim, int max_rows, hipStream_t stream);
// The 16-row-tile prefill kernel (pa_prefill16.hip), used at head size 256.
hipError_t launch_prefill16(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream);

// Inputs and outputs of the batch-metadata kernel (pa_batch.hip).
struct BatchParams {
    const int32_t *block_ids;     // packed per-request block ids
    const int32_t *block_off;     // [S+1] request s owns block_ids[block_off[s] .. block_off[s+1])
    const int32_t *num_computed;  // [S]
    const int32_t *n_new;         // [S]
    int32_t *block_tables;        // [S][max_blocks]
    int32_t *seq_lens;            // [S]
    int32_t *qsl;                 // [S+1]
    int32_t *pos;                 // [T]
    int64_t *slots;               // [T]
    int32_t *err;                 // nullable
    int32_t S, T, block_size, max_blocks, num_blocks;
};
hipError_t launch_build_batch(const BatchParams &p, hipStream_t stream);
hipError_t launch_swa_free(const int32_t *qsl, const int32_t *pos, int32_t S, int32_t T, int32_t n_swa,
                           int32_t block_size, int32_t *n_free, int32_t *block_tables, int32_t max_blocks,
                           hipStream_t stream);

// Inputs of the fused RoPE + KV write (pa_rope.hip).
struct RopeParams {
    const float *k_rows;          // [T][Hkv*D] before RoPE
    const float *v_rows;          // [T][Hkv*Dv]
    const float *q_in;            // nullable [T][H*D]
    float *q_out;                 // [T][H*D] when q_in is set (may equal q_in)
    const int32_t *pos;           // [T]
    const int64_t *slots;         // [T]
    void *k_pool, *v_pool;
    const float *freq_factors;    // nullable [n_dims/2]
    int32_t *err;
    int64_t n_cells;
    int32_t T, H, Hkv, D, Dv, n_dims, mode;
    float theta_scale, freq_scale, ext_factor, mscale, corr0, corr1;
};
hipError_t launch_rope_kv_write(const RopeParams &p, int type_k, int type_v, hipStream_t stream);

// General fp32 path (pa_general.hip): any K/V types of F32, F16, Q8_0; head
// sizes 4..512 in steps of 4; any block size.
hipError_t launch_general(const GenParams &p, int type_k, int type_v, hipStream_t stream);
size_t general_lds_bytes(int tile_cells, int D, int Dv, int rows_per_block);
int general_tile_cells(int D, int Dv);
int general_rows_per_block(int max_rows);

hipError_t launch_kv_write(const float *rows, int64_t n_rows, int64_t row_elems, const int64_t *slots, void *pool,
                           int64_t n_cells, int type, int32_t *err, hipStream_t stream);
// K and V pools of one layer over one slot list: one launch when the types match.
hipError_t launch_kv_write_kv(const float *k_rows, const float *v_rows, int64_t n_rows, int64_t k_row_elems,
                              int64_t v_row_elems, const int64_t *slots, void *k_pool, void *v_pool, int64_t n_cells,
                              int type_k, int type_v, int32_t *err, hipStream_t stream);
hipError_t launch_dequant_q8_0(const void *pool, int64_t n_cells, const int64_t *rows_idx, int64_t n_rows,
                               int64_t row_elems, float *out, hipStream_t stream);

}  // namespace iian_pa
