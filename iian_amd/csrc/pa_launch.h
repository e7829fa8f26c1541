// pa_launch.h - internal launchers shared between the kernel files and the C ABI layer.
#pragma once

#include "pa_common.h"

namespace iian_pa {

// Decode / spec-verify kernel (sequences with n_q*gqa <= p.decode_rows) plus the stream-K merge.
hipError_t launch_decode(const AttnParams &p, int head_dim, int kv_type, hipStream_t stream);
// The Q8_0-pool variant of launch_decode (pa_decode_q8.hip).
hipError_t launch_decode_q8(const AttnParams &p, int head_dim, hipStream_t stream);
// Log-sum-exp merge of the decode kernels' stream-K partial records.
hipError_t launch_merge(const AttnParams &p, int head_dim, hipStream_t stream);
// MFMA prefill kernel (sequences with n_q*gqa > p.decode_rows); grid covers max_query_len*gqa rows.
hipError_t launch_prefill(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream);
// A mixed batch over an f16 pool at head size 64 or 128 in one launch: prefill
// workgroups plus the decode rows' stream-K workers, which merge their split
// segments themselves.
hipError_t launch_mixed_f16(const AttnParams &p, int head_dim, int max_rows, hipStream_t stream);
// The 16-row-tile prefill kernel (pa_prefill16.hip), used at head size 256.
hipError_t launch_prefill16(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream);

hipError_t launch_kv_write(const float *rows, int64_t n_rows, int64_t row_elems, const int64_t *slots, void *pool,
                           int64_t n_cells, int type, int32_t *err, hipStream_t stream);
// K and V pools of one layer over one slot list: one launch when the types match.
hipError_t launch_kv_write_kv(const float *k_rows, const float *v_rows, int64_t n_rows, int64_t k_row_elems,
                              int64_t v_row_elems, const int64_t *slots, void *k_pool, void *v_pool, int64_t n_cells,
                              int type_k, int type_v, int32_t *err, hipStream_t stream);
hipError_t launch_dequant_q8_0(const void *pool, int64_t n_cells, const int64_t *rows_idx, int64_t n_rows,
                               int64_t row_elems, float *out, hipStream_t stream);

}  // namespace iian_pa
