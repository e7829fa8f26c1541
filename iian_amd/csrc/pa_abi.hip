// pa_abi.hip - extern "C" boundary of libiian_pa.so (declared in include/iian_pa.h).
//
// Host-side argument validation and launch planning; every device launch is
// asynchronous on the caller's stream.  No exceptions cross the boundary.
#include "../../include/iian_pa.h"
#include "pa_common.h"
#include "pa_launch.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <random>

namespace {

using namespace iian_pa;

// Stream-K workers of the decode kernels (for_each_piece, pa_common.h), per CU
// of the device, sized so that every worker's equal share of the call runs at
// once and the kernel ends with no tail.  The f16 kernel runs single-wave
// workgroups, 1.5 per SIMD: measured on a 256-CU MI355X at the Llama-3-8B
// decode shape, 1536 waves stream the pool fastest (127.0 us against 127.4 at
// 1280, 129.2 at 1024, 131.4 at 2048, 131.9 at 1792, 136.4 at 1152), and
// deeper per-wave prefetch gains nothing, so the pool's access pattern, not
// the number of loads in flight, sets the rate.  In a mixed launch each
// decode workgroup takes a prefill workgroup's slot on its CU while it runs
// (see kF16MixedDecodeWavesPerCu).  The Q8_0 kernel's workers are
// groups of Hkv workgroups of NW waves over 8 waves per CU: its LDS staging
// and conversion want two waves per SIMD (half of that measured 1.7x slower at
// config 4).  At head size 256 a tile moves twice the bytes and 3 waves per CU
// measured best (Gemma3-12B shapes: sliding-window layer 50.6 us against 56.6
// us at 4 per CU, 58.0 at 2.5, 60.9 at 2, 61.1 at 8; global layer 808 us
// against 824 us at 4 per CU).
constexpr int kF16DecodeWavesPerCu = 6;
// In the mixed prefill launch the decode workers' workgroups (4 waves each)
// are dispatched first and take a prefill workgroup's slot on their CU while
// they run.  With the prefill kernel as it is now, 3 waves per CU (192
// workgroups) measured best: Qwen3-8B chunked prefill + 32 decode rows 153.7
// against 155.1 us at 2 per CU, 162.9 at 4, 204.9 at 1; with one chunk of no
// prior context 147.6 against 157.1 at 2, 147.9 at 4, 208.4 at 1.
constexpr int kF16MixedDecodeWavesPerCu = 3;
constexpr int kF16DecodeWavesPerCuD256 = 3;
// Head pairs at head size 96 (two kv heads per wave, twice the bytes per
// unit of work): 4 waves per CU measured best at Phi-3.5 shapes (414 us
// against 420 at 3, 426 at 6, 455 at 2).
constexpr int kF16DecodeWavesPerCuPairs = 4;
constexpr int kQ8DecodeWavesPerCu = 8;
constexpr int kMaxWavesPerCu = kQ8DecodeWavesPerCu;
constexpr int kDefaultCus = 256;   // an MI355X, when the device cannot be queried
constexpr int kMaxHeadDim = 1024;  // largest head size the general kernel stages (pa_general.hip)
constexpr int kMaxDevices = 64;

// Compute units of device `dev`, queried once per device.
int device_cus(int dev) {
    static std::atomic<int> cache[kMaxDevices];
    if (dev < 0 || dev >= kMaxDevices) return kDefaultCus;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = kDefaultCus;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

int current_device_cus() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess ? device_cus(dev) : kDefaultCus;
}

int stream_device_cus(hipStream_t st) {
    int dev = 0;
    if (st != nullptr && hipStreamGetDevice(st, &dev) == hipSuccess) return device_cus(dev);
    return current_device_cus();
}

int q8_waves_per_wg(int decode_rows) { return decode_rows > 16 ? 2 : 1; }   // NW of pa_decode_q8_kernel

// Workspace: [partial records (numerators)][(m, l) per record row][segment
// info][merge counter per (sequence, kv head)], each section 256-byte aligned.  Sized for the record count of
// either kernel at kDecodeRowsMax rows: the f16 kernel has at most
// (f16 workers) + S*Hkv one-head records, the Q8_0 kernel at most
// (Q8_0 groups) + S records of Hkv heads; both are below
// kMaxWavesPerCu*CUs + S*Hkv heads.  A record is padded by 64 floats
// so that consecutive records do not sit at a power-of-two stride (rows at
// such strides alias onto the same HBM channels).  The general path
// (pa_general.hip) keeps its split records in the same bytes.
constexpr int kRecordPad = 64;

struct WorkspaceLayout {
    size_t o, ml, seg, ctr, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t) 255; }

WorkspaceLayout workspace_layout(int32_t n_seqs, int32_t n_head_kv, int32_t head_dim_v, int cus) {
    const size_t rec_heads = (size_t) kMaxWavesPerCu * cus + (size_t) n_seqs * n_head_kv;   // records x heads, upper bound
    WorkspaceLayout l;
    l.o = 0;
    l.ml = l.o + align256((rec_heads * kDecodeRowsMax * head_dim_v + rec_heads * kRecordPad) * sizeof(float));
    l.seg = l.ml + align256(rec_heads * kDecodeRowsMax * 2 * sizeof(float));
    l.ctr = l.seg + align256((size_t) n_seqs * n_head_kv * sizeof(int2));
    l.total = l.ctr + align256((size_t) n_seqs * n_head_kv * sizeof(uint64_t));
    return l;
}

// The bytes one call actually uses: records = workers + segments (a piece
// (worker w, segment g) writes record w + g), each rec_stride floats, with
// rec_heads * decode_rows (m, l) pairs; the segment table; a merge counter per
// (sequence, kv head).  Never more than workspace_layout's upper bound.
WorkspaceLayout exact_layout(const AttnParams &p) {
    const size_t nseg = p.rec_heads > 1 ? (size_t) p.S : (size_t) p.S * p.Hkv;
    const size_t records = (size_t) p.sk_workers + nseg;
    WorkspaceLayout l;
    l.o = 0;
    l.ml = align256(records * (size_t) p.rec_stride * sizeof(float));
    l.seg = l.ml + align256(records * p.rec_heads * p.rec_rows * 2 * sizeof(float));
    l.ctr = l.seg + align256(nseg * sizeof(int2));
    l.total = l.ctr + align256((size_t) p.S * p.Hkv * sizeof(uint64_t));
    return l;
}

// ---- Scratch of the no-allocation entry point (iian_pa_attention_noalloc) ----
//
// A file-scope device array, one copy per GPU, living until the process
// ends.  kScratchBytes covers every BASELINE configuration's call (the
// largest, Q8_0 spec-verify at 128 sequences x 8 kv heads, uses 34 MB).  On
// the host, `scratch` names a stand-in, not device memory: its device
// address is taken once per device with hipGetSymbolAddress (with that
// device current) and only that address is ever handed to kernels.
constexpr size_t kScratchBytes = (size_t) 64 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

// Device address of `scratch` on device dev (nullptr when it cannot be taken).
char *scratch_address(int dev) {
    static std::atomic<char *> addr[kMaxDevices];
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    char *a = addr[dev].load(std::memory_order_acquire);
    if (a) return a;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return nullptr;
    if (e != hipSuccess || !ptr) return nullptr;
    addr[dev].store((char *) ptr, std::memory_order_release);
    return (char *) ptr;
}

// Where a call's workspace comes from: the caller's buffer (iian_pa_attention;
// at least iian_pa_workspace_size bytes, any alignment) or the library's
// scratch on the stream's device (iian_pa_attention_noalloc).
struct WsSource {
    void *base;
    size_t bytes;
    bool scratch;
};

// 256-aligned base of `need` bytes of the call's workspace, or a status.
int ws_resolve(const WsSource &src, hipStream_t st, size_t need, char **ws) {
    if (!src.scratch) {
        const char *b = (const char *) (((uintptr_t) src.base + 255) & ~(uintptr_t) 255);
        if (need > src.bytes - (size_t) (b - (const char *) src.base)) return IIAN_PA_ERR_WORKSPACE;
        *ws = (char *) b;
        return IIAN_PA_OK;
    }
    if (need > kScratchBytes) return IIAN_PA_ERR_SCRATCH;
    int dev = 0;
    if (st != nullptr ? hipStreamGetDevice(st, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess)
        return IIAN_PA_ERR_HIP;
    char *a = scratch_address(dev);
    if (!a) return IIAN_PA_ERR_HIP;
    *ws = a;
    return IIAN_PA_OK;
}

// Tags of the mixed launch's merge counters: one per call, 48 bits, counting
// up from a random start, so that workspace bytes the library never wrote
// pass for a counter of the current call only with probability 2^-48 per
// counter (the kernel treats any other tag as a count of zero).
uint64_t next_epoch() {
    static std::atomic<uint64_t> next{[] {
        uint64_t seed = (uint64_t) std::chrono::steady_clock::now().time_since_epoch().count() * 0x9e3779b97f4a7c15ull;
        seed ^= (uint64_t) (uintptr_t) &seed;
        try {   // no exception may leave the C ABI; the clock alone still seeds
            std::random_device rd;
            seed ^= (uint64_t) rd() << 32 ^ (uint64_t) rd();
        } catch (...) {
        }
        return seed;
    }()};
    return next.fetch_add(1, std::memory_order_relaxed) & ((1ull << 48) - 1);
}

// Side stream and fork/join events of one host thread for one device, created
// on first use (default priority, non-blocking) and kept for the life of the
// process.  Per thread, so concurrent callers never share an event.
struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};

const SideStream *side_stream_for(hipStream_t caller) {
    int dev = 0;
    if (hipStreamGetDevice(caller, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    thread_local SideStream slots[kMaxDevices];
    SideStream &s = slots[dev];
    if (s.join) return &s;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    bool ok = (s.stream || hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) == hipSuccess) &&
              (s.fork || hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) == hipSuccess) &&
              hipEventCreateWithFlags(&s.join, hipEventDisableTiming) == hipSuccess;
    if (!ok) s.join = nullptr;
    if (cur != dev && hipSetDevice(cur) != hipSuccess) ok = false;
    return ok ? &s : nullptr;
}

int log2_exact(int32_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int l = 0;
    while ((1 << l) < v) l++;
    return l;
}

int row_bytes(int type, int64_t elems, int64_t &out) {
    switch (type) {
        case IIAN_PA_TYPE_F32: out = elems * 4; return 0;
        case IIAN_PA_TYPE_F16: out = elems * 2; return 0;
        case IIAN_PA_TYPE_Q8_0:
            if (elems % 32) return IIAN_PA_ERR_ARG;
            out = elems / 32 * 34;
            return 0;
        default: return IIAN_PA_ERR_UNSUPPORTED;
    }
}

// The MFMA kernels: K and V both f16 or both Q8_0, head size 64, 128 or 256
// for both, and a power-of-two block size of at least 8 (the 8-cell groups of
// a tile must not straddle a block); f16 pools at head size 96 too (run_attention
// checks those itself).  Everything else iian_pa_supported accepts runs
// through the general fp32 kernel.
bool mfma_path(int type_k, int type_v, int head_dim, int head_dim_v, int bs_log2) {
    return type_k == type_v && (type_k == IIAN_PA_TYPE_F16 || type_k == IIAN_PA_TYPE_Q8_0) &&
           head_dim == head_dim_v && (head_dim == 64 || head_dim == 128 || head_dim == 256) && bs_log2 >= 3;
}

// Any head size the general kernel stages (1 .. 1024; the reference's op
// takes any, paged_attn.cpp:96-100); a Q8_0 head slice is whole 32-value
// blocks.
bool head_size_ok(int type, int d) {
    if (d < 1 || d > kMaxHeadDim) return false;
    return type != IIAN_PA_TYPE_Q8_0 || d % 32 == 0;
}

}  // namespace

extern "C" {

const char *iian_pa_status_string(int status) {
    switch (status) {
        case IIAN_PA_OK: return "ok";
        case IIAN_PA_ERR_NULL: return "a required pointer is NULL";
        case IIAN_PA_ERR_ARG: return "invalid or inconsistent sizes";
        case IIAN_PA_ERR_UNSUPPORTED: return "unsupported KV type, head size or ALiBi";
        case IIAN_PA_ERR_WORKSPACE: return "workspace missing or too small";
        case IIAN_PA_ERR_HIP: return "HIP runtime error";
        case IIAN_PA_ERR_SCRATCH: return "the call needs more than the library's 64 MiB scratch (iian_pa_attention_noalloc)";
        default: return "unknown status";
    }
}

int iian_pa_supported(int type_k, int type_v, int head_dim, int head_dim_v, float max_alibi_bias) {
    if (max_alibi_bias != 0.0f) return 0;
    auto type_ok = [](int t) { return t == IIAN_PA_TYPE_F32 || t == IIAN_PA_TYPE_F16 || t == IIAN_PA_TYPE_Q8_0; };
    if (!type_ok(type_k) || !type_ok(type_v)) return 0;
    return head_size_ok(type_k, head_dim) && head_size_ok(type_v, head_dim_v);
}

int iian_pa_kv_write(void *stream, const float *rows, int64_t n_rows, int64_t row_elems, const int64_t *slots,
                     void *pool, int64_t n_cells, int type, int32_t *err_flag) {
    if (n_rows < 0 || row_elems <= 0 || n_cells < 0) return IIAN_PA_ERR_ARG;
    if (n_rows == 0) return IIAN_PA_OK;
    if (!rows || !slots || !pool) return IIAN_PA_ERR_NULL;
    int64_t rb;
    const int rc = row_bytes(type, row_elems, rb);
    if (rc) return rc;
    const hipError_t e = launch_kv_write(rows, n_rows, row_elems, slots, pool, n_cells, type, err_flag,
                                         (hipStream_t) stream);
    return e == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

int iian_pa_kv_write_kv(void *stream, const float *k_rows, const float *v_rows, int64_t n_rows,
                        int64_t k_row_elems, int64_t v_row_elems, const int64_t *slots, void *k_pool, void *v_pool,
                        int64_t n_cells, int type_k, int type_v, int32_t *err_flag) {
    if (n_rows < 0 || k_row_elems <= 0 || v_row_elems <= 0 || n_cells < 0) return IIAN_PA_ERR_ARG;
    if (n_rows == 0) return IIAN_PA_OK;
    if (!k_rows || !v_rows || !slots || !k_pool || !v_pool) return IIAN_PA_ERR_NULL;
    int64_t kb, vb;
    int rc = row_bytes(type_k, k_row_elems, kb);
    if (rc) return rc;
    rc = row_bytes(type_v, v_row_elems, vb);
    if (rc) return rc;
    const hipError_t e = launch_kv_write_kv(k_rows, v_rows, n_rows, k_row_elems, v_row_elems, slots, k_pool, v_pool,
                                            n_cells, type_k, type_v, err_flag, (hipStream_t) stream);
    return e == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

size_t iian_pa_workspace_size(int32_t n_tokens, int32_t n_seqs, int32_t n_head, int32_t n_head_kv,
                              int32_t head_dim_v, int32_t max_blocks, int32_t block_size) {
    if (n_tokens < 0 || n_seqs < 0 || n_head <= 0 || n_head_kv <= 0 || head_dim_v <= 0 || max_blocks < 0 ||
        block_size <= 0)
        return 0;
    // + 256: room to align the caller's base to 256 bytes
    return workspace_layout(n_seqs, n_head_kv, head_dim_v, current_device_cus()).total + 256;
}

}  // extern "C"

namespace {

// The attention call behind iian_pa_attention and iian_pa_attention_noalloc,
// on the workspace `src` names.
int run_attention(hipStream_t st, const float *q, const void *k_pool, const void *v_pool, int type_k, int type_v,
                  int32_t num_blocks, const int32_t *block_tables, int32_t max_blocks, const int32_t *seq_lens,
                  const int32_t *query_start_loc, const int32_t *pos, int32_t n_tokens, int32_t n_seqs,
                  int32_t max_query_len, int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t head_dim_v,
                  int32_t block_size, float scale, float softcap, int32_t causal, int32_t n_swa, float *out,
                  const WsSource &src, int32_t *err_flag, const float *k_new = nullptr,
                  const float *v_new = nullptr) {
    if (n_tokens < 0 || n_seqs < 0 || max_query_len < 0) return IIAN_PA_ERR_ARG;
    if (n_tokens == 0 || n_seqs == 0) return IIAN_PA_OK;
    if (!q || !k_pool || !v_pool || !block_tables || !seq_lens || !query_start_loc || !pos || !out)
        return IIAN_PA_ERR_NULL;
    const bool write_new = k_new || v_new;   // iian_pa_write_attention
    if (write_new && (!k_new || !v_new)) return IIAN_PA_ERR_NULL;
    if (((uintptr_t) k_new | (uintptr_t) v_new) & 15) return IIAN_PA_ERR_ARG;
    if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv) return IIAN_PA_ERR_ARG;
    if (num_blocks <= 0 || max_blocks <= 0 || block_size <= 0 || max_query_len == 0 || max_query_len > n_tokens)
        return IIAN_PA_ERR_ARG;
    if (n_swa < 0 || softcap < 0.0f || !std::isfinite(scale) || !std::isfinite(softcap)) return IIAN_PA_ERR_ARG;
    if (!iian_pa_supported(type_k, type_v, head_dim, head_dim_v, 0.0f)) return IIAN_PA_ERR_UNSUPPORTED;
    if (((uintptr_t) q | (uintptr_t) k_pool | (uintptr_t) v_pool | (uintptr_t) out) & 15) return IIAN_PA_ERR_ARG;
    const int cus = stream_device_cus(st);
    const WorkspaceLayout wl = workspace_layout(n_seqs, n_head_kv, head_dim_v, cus);
    // a caller's workspace must hold iian_pa_workspace_size bytes, whatever this call uses
    if (!src.scratch && (!src.base || src.bytes < wl.total + 256)) return IIAN_PA_ERR_WORKSPACE;
    char *ws = nullptr;
    int64_t kr, vr;
    if (row_bytes(type_k, (int64_t) n_head_kv * head_dim, kr) || row_bytes(type_v, (int64_t) n_head_kv * head_dim_v, vr))
        return IIAN_PA_ERR_ARG;
    const int bs_log2 = log2_exact(block_size);
    const int gqa = n_head / n_head_kv;

    // f16 pools at head size 96 (Phi-3) take the MFMA kernels too: the decode
    // kernel when every sequence of the call is a decode or spec-verify row
    // set, the mixed prefill launch otherwise
    const bool f16_96 = type_k == IIAN_PA_TYPE_F16 && type_v == IIAN_PA_TYPE_F16 && head_dim == 96 &&
                        head_dim_v == 96 && bs_log2 >= 3;
    const bool decode96 = f16_96 && (int64_t) max_query_len * gqa <= kDecodeRowsMax;
    // the fused KV write lives in the f16 decode kernels: f16 pools, one head
    // size for K and V, every sequence of the call a decode or spec-verify row set
    if (write_new && (type_k != IIAN_PA_TYPE_F16 || type_v != IIAN_PA_TYPE_F16 || head_dim != head_dim_v ||
                      (int64_t) max_query_len * gqa > kDecodeRowsMax ||
                      !(mfma_path(type_k, type_v, head_dim, head_dim_v, bs_log2) || f16_96)))
        return IIAN_PA_ERR_UNSUPPORTED;
    if (!mfma_path(type_k, type_v, head_dim, head_dim_v, bs_log2) && !f16_96) {
        // General fp32 path.  Cell indices within a sequence and pool rows
        // are int32 / int64 there.
        if ((int64_t) max_blocks * block_size > INT32_MAX) return IIAN_PA_ERR_UNSUPPORTED;
        GenParams g = {};
        g.q = q;
        g.k_pool = (const char *) k_pool;
        g.v_pool = (const char *) v_pool;
        g.bt = block_tables;
        g.seq_lens = seq_lens;
        g.qsl = query_start_loc;
        g.pos = pos;
        g.out = out;
        g.err = err_flag;
        g.k_row = kr;
        g.v_row = vr;
        g.max_blocks = max_blocks;
        g.num_blocks = num_blocks;
        g.block_size = block_size;
        g.T = n_tokens;
        g.S = n_seqs;
        g.H = n_head;
        g.Hkv = n_head_kv;
        g.gqa = gqa;
        g.D = head_dim;
        g.Dv = head_dim_v;
        g.max_q = max_query_len;
        g.scale = scale;
        g.softcap = softcap;
        g.causal = causal ? 1 : 0;
        g.n_swa = n_swa;
        g.tile_cells = general_tile_cells(head_dim, head_dim_v);
        const int rows = general_rows_per_block((int) std::min<int64_t>((int64_t) max_query_len * gqa, INT32_MAX));
        g.rows_per_block = rows;
        g.n_rb = (int) (((int64_t) max_query_len * gqa + rows - 1) / rows);
        // Split each row block's KV range until the launch holds about 8
        // workgroups per CU (16 for 4-row workgroups: cfg2's shape with F32
        // pools ran 396 against 471 us), keeping at least 2 tiles per range of the
        // longest sequence the tables can hold, and the records inside the
        // workspace: [T*H][n_split] rows of (Dv floats) + (m, l).  The
        // no-allocation entry point's workspace is the scratch array, so its
        // records must also fit kScratchBytes (one range needs none).
        const int64_t base = (int64_t) n_seqs * n_head_kv * g.n_rb;
        const int64_t max_tiles = ((int64_t) max_blocks * block_size + g.tile_cells - 1) / g.tile_cells;
        int64_t ns = ((rows == 4 ? 16LL : 8LL) * cus + base - 1) / base;
        ns = std::min<int64_t>(ns, std::max<int64_t>(1, max_tiles / 2));
        ns = std::min<int64_t>(ns, 64);
        // record rows are Dv rounded up to a multiple of 4 floats
        const size_t dv4 = (size_t) (head_dim_v + 3) & ~(size_t) 3;
        const size_t per_split = (size_t) n_tokens * n_head * (dv4 + 2) * sizeof(float) + 512;
        const size_t rec_cap = src.scratch ? std::min(wl.total, kScratchBytes) : wl.total;
        ns = std::min<int64_t>(ns, (int64_t) (rec_cap / per_split));
        g.n_split = (int) std::max<int64_t>(ns, 1);
        const size_t o_bytes = align256((size_t) n_tokens * n_head * g.n_split * dv4 * sizeof(float));
        const size_t need = g.n_split > 1 ? o_bytes + (size_t) n_tokens * n_head * g.n_split * 2 * sizeof(float) : 0;
        const int rc = ws_resolve(src, st, need, &ws);
        if (rc) return rc;
        g.part_o = (float *) ws;
        g.part_ml = (float *) (ws + o_bytes);
        return launch_general(g, type_k, type_v, st) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
    }

    AttnParams p = {};
    p.q = q;
    p.k_pool = (const char *) k_pool;
    p.v_pool = (const char *) v_pool;
    p.bt = block_tables;
    p.seq_lens = seq_lens;
    p.qsl = query_start_loc;
    p.pos = pos;
    p.out = out;
    p.err = err_flag;
    // The kernels index pool rows with 32-bit cell numbers and row lengths
    // (pool_off): 2^32 cells of the smallest supported row (68 bytes, one
    // Q8_0 head of size 64) are 272 GiB, more than an MI355X's 288 GB hold.
    // Rows stay below 1 GiB, so that a prefill DMA lane's byte offset within
    // the 4 rows of its instruction fits 32 bits.
    if (((int64_t) num_blocks << bs_log2) > ((int64_t) 1 << 32) || kr != vr || kr >= ((int64_t) 1 << 30))
        return IIAN_PA_ERR_UNSUPPORTED;
    p.k_row = kr;
    p.v_row = vr;
    p.max_blocks = max_blocks;
    p.num_blocks = num_blocks;
    p.T = n_tokens;
    p.S = n_seqs;
    p.H = n_head;
    p.Hkv = n_head_kv;
    p.gqa = gqa;
    p.bs_log2 = bs_log2;
    p.softcap = softcap;
    p.softcap_inv = softcap > 0.0f ? 1.0f / softcap : 0.0f;
    // exp2-domain softmax: fold log2(e) into q unless the softcap has to see the raw score first
    p.qscale = softcap > 0.0f ? scale : scale * kLog2e;
    p.causal = causal ? 1 : 0;
    p.n_swa = n_swa;
    p.max_q = max_query_len;
    p.cus_per_xcd = std::max(1, cus / 8);
    // Row budget of the decode kernel: one 16-row MFMA tile, or two when that
    // covers every sequence of the call (spec-verify); larger sequences go to
    // the prefill kernel.
    const int max_rows = max_query_len * p.gqa;
    p.decode_rows = (max_rows > 16 && max_rows <= kDecodeRowsMax) ? kDecodeRowsMax : 16;
    // f16 decode at head size 96: one wave per pair of kv heads (their slices
    // of a cell row are three whole 128-byte lines; one head's slice shares a
    // line with its neighbour's) when every sequence has at most 8 rows per kv
    // head, so that a pair's rows fill one 16-row tile
    p.head_group = 1;
    if (decode96 && max_rows <= 8 && n_head_kv % 2 == 0) {
        p.head_group = 2;
        p.decode_rows = 8;
    }

    if (type_k == IIAN_PA_TYPE_Q8_0) {
        p.rec_heads = n_head_kv;
        p.sk_workers = std::max(1, kQ8DecodeWavesPerCu * cus / (q8_waves_per_wg(p.decode_rows) * n_head_kv));
    } else {
        p.rec_heads = 1;
        p.sk_workers = (head_dim == 256 ? kF16DecodeWavesPerCuD256 : kF16DecodeWavesPerCu) * cus;
        if (p.head_group == 2) p.sk_workers = kF16DecodeWavesPerCuPairs * cus;
    }
    p.rec_rows = p.decode_rows * p.head_group;
    p.rec_stride = (int64_t) p.rec_heads * p.rec_rows * head_dim_v + kRecordPad;
    const bool decode_only = max_rows <= p.decode_rows;
    if (write_new && !decode_only) return IIAN_PA_ERR_UNSUPPORTED;
    p.k_new = k_new;
    p.v_new = v_new;
    // f16 decode calls with short or window-bounded segments: one workgroup
    // per (sequence, kv head) attends and merges in LDS, in one launch
    // (pa_decode_seg_kernel).  With no sliding window, when the block-table
    // width leaves no segment more than two tiles per wave of a segment
    // workgroup; with one, when a decode step's window (n_swa cells plus the
    // query span, tile-aligned) keeps every wave within kSegSwaTilesPerWave
    // tiles and the call has a segment for every CU.
    if (decode_only && type_k == IIAN_PA_TYPE_F16 && p.decode_rows == 16 &&
        (head_dim == 64 || head_dim == 128 || head_dim == 256)) {
        const int sw = head_dim == 64 ? kSegWavesD64 : head_dim == 128 ? kSegWavesD128 : kSegWavesD256;
        const int64_t tiles = (((int64_t) max_blocks << bs_log2) + kTile - 1) / kTile;
        if (n_swa <= 0) {
            if (tiles <= 2 * sw) p.seg_waves = sw;
        } else {
            const int64_t wtiles = std::min<int64_t>(tiles, ((int64_t) n_swa + max_query_len - 1 + 2 * kTile - 2) / kTile);
            if (wtiles <= (int64_t) kSegSwaTilesPerWave * sw && (int64_t) n_seqs * n_head_kv >= cus) p.seg_waves = sw;
        }
    }
    // Mixed batch over an f16 pool (head size 64, 96 or 128): one launch holds the
    // prefill workgroups and, after them, the decode rows' stream-K workers,
    // which fill the CUs the MFMA-bound prefill leaves, and merge their split
    // segments themselves.
    const bool mixed_one_launch = !decode_only && type_k == IIAN_PA_TYPE_F16 && head_dim <= 128;
    // No sequence can be a decode row when even the smallest possible query
    // count, T - (S - 1) * max_query_len (the others holding at most
    // max_query_len each), is above the decode row budget: then no decode
    // worker or decode launch is issued at all, and the row budget drops to
    // 0 so that the prefill kernel covers every sequence.  (A max_query_len
    // below the batch's largest query count, flagged by bit 2, can break the
    // bound; a decode sequence is then attended by the prefill kernel, not
    // left unwritten.)
    const bool no_decode_rows =
        !decode_only && ((int64_t) n_tokens - (int64_t) (n_seqs - 1) * max_query_len) * gqa > p.decode_rows;
    if (mixed_one_launch) p.sk_workers = kF16MixedDecodeWavesPerCu * cus;
    if (no_decode_rows) {
        p.decode_rows = 0;
        p.sk_workers = 0;
    }
    const WorkspaceLayout xl = exact_layout(p);
    const int rc = ws_resolve(src, st, xl.total, &ws);
    if (rc) return rc;
    p.part_o = (float *) (ws + xl.o);
    p.part_ml = (float *) (ws + xl.ml);
    p.seg_info = (int2 *) (ws + xl.seg);
    p.seg_ctr = (uint64_t *) (ws + xl.ctr);
    p.epoch = next_epoch();
    if (decode_only) return launch_decode(p, head_dim, type_k, st) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
    if (mixed_one_launch)
        return launch_mixed_f16(p, head_dim, max_rows, st) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;

    // Other mixed batches: the decode rows (HBM-bound) run on a side stream
    // forked from and joined back into the caller's stream, beside the
    // MFMA-bound prefill kernel, which fills the CUs first and leaves its tail
    // to the decode waves.  The no-allocation entry point creates no stream:
    // it runs both kernels in order on the caller's stream.
    if (no_decode_rows)
        return launch_prefill(p, head_dim, type_k, max_rows, st) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
    if (src.scratch) {
        if (launch_prefill(p, head_dim, type_k, max_rows, st) != hipSuccess) return IIAN_PA_ERR_HIP;
        return launch_decode(p, head_dim, type_k, st) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
    }
    const SideStream *side = side_stream_for(st);
    if (!side) return IIAN_PA_ERR_HIP;
    if (hipEventRecord(side->fork, st) != hipSuccess || hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)
        return IIAN_PA_ERR_HIP;
    if (launch_prefill(p, head_dim, type_k, max_rows, st) != hipSuccess) return IIAN_PA_ERR_HIP;
    const hipError_t ed = launch_decode(p, head_dim, type_k, side->stream);
    // join even when the decode launch failed, so the caller's stream never
    // runs ahead of work queued on the side stream
    if (hipEventRecord(side->join, side->stream) != hipSuccess || hipStreamWaitEvent(st, side->join, 0) != hipSuccess)
        return IIAN_PA_ERR_HIP;
    return ed == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

}  // namespace

extern "C" {

int iian_pa_attention(void *stream, const float *q, const void *k_pool, const void *v_pool, int type_k, int type_v,
                      int32_t num_blocks, const int32_t *block_tables, int32_t max_blocks, const int32_t *seq_lens,
                      const int32_t *query_start_loc, const int32_t *pos, int32_t n_tokens, int32_t n_seqs,
                      int32_t max_query_len, int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t head_dim_v,
                      int32_t block_size, float scale, float softcap, int32_t causal, int32_t n_swa, float *out,
                      void *workspace, size_t workspace_bytes, int32_t *err_flag) {
    const WsSource src = {workspace, workspace_bytes, false};
    return run_attention((hipStream_t) stream, q, k_pool, v_pool, type_k, type_v, num_blocks, block_tables,
                         max_blocks, seq_lens, query_start_loc, pos, n_tokens, n_seqs, max_query_len, n_head,
                         n_head_kv, head_dim, head_dim_v, block_size, scale, softcap, causal, n_swa, out, src,
                         err_flag);
}

int iian_pa_attention_noalloc(void *stream, const float *q, const void *k_pool, const void *v_pool, int type_k,
                              int type_v, int32_t num_blocks, const int32_t *block_tables, int32_t max_blocks,
                              const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *pos,
                              int32_t n_tokens, int32_t n_seqs, int32_t max_query_len, int32_t n_head,
                              int32_t n_head_kv, int32_t head_dim, int32_t head_dim_v, int32_t block_size, float scale,
                              float softcap, int32_t causal, int32_t n_swa, float *out, int32_t *err_flag) {
    const WsSource src = {nullptr, kScratchBytes, true};
    return run_attention((hipStream_t) stream, q, k_pool, v_pool, type_k, type_v, num_blocks, block_tables,
                         max_blocks, seq_lens, query_start_loc, pos, n_tokens, n_seqs, max_query_len, n_head,
                         n_head_kv, head_dim, head_dim_v, block_size, scale, softcap, causal, n_swa, out, src,
                         err_flag);
}

int iian_pa_write_attention(void *stream, const float *q, const float *k_new, const float *v_new, void *k_pool,
                            void *v_pool, int type_k, int type_v, int32_t num_blocks, const int32_t *block_tables,
                            int32_t max_blocks, const int32_t *seq_lens, const int32_t *query_start_loc,
                            const int32_t *pos, int32_t n_tokens, int32_t n_seqs, int32_t max_query_len,
                            int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t head_dim_v,
                            int32_t block_size, float scale, float softcap, int32_t causal, int32_t n_swa, float *out,
                            void *workspace, size_t workspace_bytes, int32_t *err_flag) {
    if (n_tokens > 0 && n_seqs > 0 && (!k_new || !v_new)) return IIAN_PA_ERR_NULL;
    const WsSource src = {workspace, workspace_bytes, false};
    return run_attention((hipStream_t) stream, q, k_pool, v_pool, type_k, type_v, num_blocks, block_tables,
                         max_blocks, seq_lens, query_start_loc, pos, n_tokens, n_seqs, max_query_len, n_head,
                         n_head_kv, head_dim, head_dim_v, block_size, scale, softcap, causal, n_swa, out, src,
                         err_flag, k_new, v_new);
}

int iian_pa_build_batch(void *stream, const int32_t *block_ids, const int32_t *block_off,
                        const int32_t *num_computed, const int32_t *n_new, int32_t n_seqs, int32_t n_tokens,
                        int32_t block_size, int32_t max_blocks, int32_t num_blocks, int32_t *block_tables,
                        int32_t *seq_lens, int32_t *query_start_loc, int32_t *pos, int64_t *slots,
                        int32_t *err_flag) {
    if (n_seqs < 0 || n_tokens < 0 || block_size <= 0 || max_blocks <= 0 || num_blocks <= 0) return IIAN_PA_ERR_ARG;
    if (n_seqs == 0) return IIAN_PA_OK;
    if (!block_off || !num_computed || !n_new || !block_tables || !seq_lens || !query_start_loc ||
        (n_tokens > 0 && (!pos || !slots)))
        return IIAN_PA_ERR_NULL;
    BatchParams p = {};
    p.block_ids = block_ids;
    p.block_off = block_off;
    p.num_computed = num_computed;
    p.n_new = n_new;
    p.block_tables = block_tables;
    p.seq_lens = seq_lens;
    p.qsl = query_start_loc;
    p.pos = pos;
    p.slots = slots;
    p.err = err_flag;
    p.S = n_seqs;
    p.T = n_tokens;
    p.block_size = block_size;
    p.max_blocks = max_blocks;
    p.num_blocks = num_blocks;
    return launch_build_batch(p, (hipStream_t) stream) == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

int iian_pa_swa_free_blocks(void *stream, const int32_t *query_start_loc, const int32_t *pos, int32_t n_seqs,
                            int32_t n_tokens, int32_t n_swa, int32_t block_size, int32_t *n_free,
                            int32_t *block_tables, int32_t max_blocks) {
    if (n_seqs < 0 || n_tokens < 0 || n_swa < 0 || block_size <= 0 || (block_tables && max_blocks <= 0))
        return IIAN_PA_ERR_ARG;
    if (n_seqs == 0) return IIAN_PA_OK;
    if (!query_start_loc || !n_free || (n_tokens > 0 && !pos)) return IIAN_PA_ERR_NULL;
    const hipError_t e = launch_swa_free(query_start_loc, pos, n_seqs, n_tokens, n_swa, block_size, n_free,
                                         block_tables, max_blocks, (hipStream_t) stream);
    return e == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

int iian_pa_rope_kv_write(void *stream, const float *k_rows, const float *v_rows, const float *q_in, float *q_out,
                          const int32_t *pos, const int64_t *slots, int64_t n_rows, int32_t n_head, int32_t n_head_kv,
                          int32_t head_dim, int32_t head_dim_v, const iian_pa_rope_params *rope, void *k_pool,
                          void *v_pool, int64_t n_cells, int type_k, int type_v, int32_t *err_flag) {
#pragma clang fp contract(off)
    if (n_rows < 0 || n_cells < 0 || n_head < 0 || n_head_kv <= 0 || head_dim <= 0 || head_dim_v <= 0)
        return IIAN_PA_ERR_ARG;
    if (n_rows == 0) return IIAN_PA_OK;
    if (!k_rows || !v_rows || !pos || !slots || !rope || !k_pool || !v_pool) return IIAN_PA_ERR_NULL;
    if ((q_in == nullptr) != (q_out == nullptr) || (q_in && n_head <= 0)) return IIAN_PA_ERR_ARG;
    if (n_rows > INT32_MAX) return IIAN_PA_ERR_ARG;
    if (rope->mode != 0 && rope->mode != 2) return IIAN_PA_ERR_UNSUPPORTED;
    if (rope->n_dims <= 0 || rope->n_dims % 2 || rope->n_dims > head_dim || head_dim % 2 || head_dim_v % 2 ||
        !(rope->freq_base > 0.0f) || !(rope->freq_scale > 0.0f))
        return IIAN_PA_ERR_ARG;
    int64_t kb, vb;
    int rc = row_bytes(type_k, (int64_t) n_head_kv * head_dim, kb);
    if (rc) return rc;
    rc = row_bytes(type_v, (int64_t) n_head_kv * head_dim_v, vb);
    if (rc) return rc;
    if ((int64_t) n_head_kv * head_dim > INT32_MAX / 2 || (int64_t) n_head_kv * head_dim_v > INT32_MAX / 2 ||
        (int64_t) n_head * head_dim > INT32_MAX / 2)
        return IIAN_PA_ERR_ARG;
    // pairs of adjacent f32 values are loaded and stored as one 8-byte access
    if (((uintptr_t) k_rows | (uintptr_t) v_rows | (uintptr_t) q_in | (uintptr_t) q_out | (uintptr_t) k_pool |
         (uintptr_t) v_pool) & 7)
        return IIAN_PA_ERR_ARG;
    // pairs of values move as 8-byte accesses: rows of an odd head size are not 8-byte aligned
    if ((head_dim | head_dim_v) & 1) return IIAN_PA_ERR_UNSUPPORTED;
    // a Q8_0 head row is quantised in its own 32-value blocks, staged whole (at most 512 values)
    if ((type_k == IIAN_PA_TYPE_Q8_0 && (head_dim % 32 || head_dim > 512)) ||
        (type_v == IIAN_PA_TYPE_Q8_0 && (head_dim_v % 32 || head_dim_v > 512)))
        return IIAN_PA_ERR_UNSUPPORTED;
    if (rope->n_dims > 512) return IIAN_PA_ERR_UNSUPPORTED;   // the (cos, sin) table: one pair per thread of 256
    RopeParams p = {};
    p.k_rows = k_rows;
    p.v_rows = v_rows;
    p.q_in = q_in;
    p.q_out = q_out;
    p.pos = pos;
    p.slots = slots;
    p.k_pool = k_pool;
    p.v_pool = v_pool;
    p.freq_factors = rope->freq_factors;
    p.err = err_flag;
    p.n_cells = n_cells;
    p.T = (int32_t) n_rows;
    p.H = n_head;
    p.Hkv = n_head_kv;
    p.D = head_dim;
    p.Dv = head_dim_v;
    p.n_dims = rope->n_dims;
    p.mode = rope->mode;
    // the per-call constants of ggml's CPU rope, computed as it computes them
    // on its host (ggml-cpu/ops.cpp:6144-6146, 5969; ggml.c:4418-4430)
    p.theta_scale = powf(rope->freq_base, -2.0f / rope->n_dims);
    const int n_dims = rope->n_dims;
    const float start = floorf(n_dims * logf(rope->n_ctx_orig / (rope->beta_fast * 2 * (float) M_PI)) /
                               (2 * logf(rope->freq_base)));
    const float end = ceilf(n_dims * logf(rope->n_ctx_orig / (rope->beta_slow * 2 * (float) M_PI)) /
                            (2 * logf(rope->freq_base)));
    p.corr0 = std::max(0.0f, start);
    p.corr1 = std::min((float) (n_dims - 1), end);
    p.freq_scale = rope->freq_scale;
    p.ext_factor = rope->ext_factor;
    p.mscale = rope->attn_factor;
    if (rope->ext_factor != 0.0f) p.mscale *= 1.0f + 0.1f * logf(1.0f / rope->freq_scale);
    const hipError_t e = launch_rope_kv_write(p, type_k, type_v, (hipStream_t) stream);
    return e == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

int iian_pa_dequant_q8_0(void *stream, const void *pool, int64_t n_cells, const int64_t *rows_idx, int64_t n_rows,
                         int64_t row_elems, float *out) {
    if (n_rows < 0 || row_elems <= 0 || row_elems % 32 || n_cells < 0) return IIAN_PA_ERR_ARG;
    if (n_rows == 0) return IIAN_PA_OK;
    if (!pool || !rows_idx || !out) return IIAN_PA_ERR_NULL;
    const hipError_t e = launch_dequant_q8_0(pool, n_cells, rows_idx, n_rows, row_elems, out, (hipStream_t) stream);
    return e == hipSuccess ? IIAN_PA_OK : IIAN_PA_ERR_HIP;
}

}  // extern "C"
