// Fused cache write of one layer step: the code projection hidden @ kv_down^T, then the
// bf16/fp16 scatter or the 3.2-bit quantize + scatter.
//
// Reference: the model's code GEMM (starkv_serve/model.py:71: kv = F.linear(hidden,
// kv_down), kv_down = [k_down; v_down], attention.py:161) and the cache write of
// StarKVAttentionImpl.forward (attention.py:179-188: cat + index_put into the bf16/fp16
// cache, or pack_kv into the 3.2-bit cache, paged_quant.py:205-216).
//
// 1. kv_gemm_kernel: split-K partial products. Workgroup (code tile t of 64, K split s,
//    token block of 64) has 4 waves; wave w takes codes [64 t + 16 w, +16) and the
//    block's tokens in 16-row MFMA tiles over split s with v_mfma_f32_16x16x32 (A = 16
//    hidden rows x 32 channels, B = 32 channels x 16 kv_down rows; channels in an order
//    that reads whole 128-byte lines), and writes fp32 partials [s][token][code]. kv_down (the layer's only large operand) is read once,
//    spread over ~256+ workgroups.
// 2. kv_store_kernel: one workgroup per token sums its partials in split order, rounds
//    every code to the model dtype (the dtype F.linear returns, round-to-nearest-even),
//    optionally writes the rounded codes out, and stores the row: the codes themselves
//    (bf16/fp16 cache) or the packed 3.2-bit row, the packers reading the rounded codes
//    from LDS exactly as pack_kv reads them from memory. For at most 16 tokens of a
//    3.2-bit cache, `groups` workgroups per token (each forming the codes) share its H K
//    blocks and V block, one block per wave.
// One token (hidden a multiple of 512, at most 4096) or two (hidden 4096) take the direct form
// instead (kv_gemm.hpp): kv_direct_kernel's workgroups own whole codes and store the
// bf16/fp16 row, or pack the 3.2-bit K blocks; a 3.2-bit row's V latent then takes
// kv_vpack_kernel (or, for a deferred write, the next decode's logits pass). Against
// the split form at one 16K-token layer step (hidden 4096, 2170 codes) it drops the
// store launch.
#include <algorithm>

#include "kv_gemm.hpp"

namespace starkv {

constexpr int KVS_THR = 1024;   // store workgroup (one token)

template <int DT>
__global__ __launch_bounds__(KVW_THR) void kv_gemm_kernel(const KvGemmParams p) {
    kv_gemm_block<DT>(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

struct KvStoreParams {
    const float* part; int splits, n, width;
    int k_width, v_rank;
    uint16_t* codes; int64_t co_s0;  // optional [n, width] rounded codes
    void* cache; int64_t c_s0, c_s1;  // element strides (bytes for the 3.2-bit cache)
    int block_size; int64_t num_blocks;
    const void* slots; int slot_bits;
    int quant;                        // 1: 3.2-bit rows
    int H; const int32_t* ranks; const int32_t* offsets; const int32_t* nouts;
    RowLayout row;
    int groups;                       // 3.2-bit rows: workgroups per token (grid.y) sharing its H + 1 blocks
};

template <int DT, int TOK, int SL>
__global__ __launch_bounds__(KVW_THR) void kv_direct_kernel(const KvDirectParams p) {
    kv_direct_block<DT, TOK, SL>(p, blockIdx.x);
}

// The V latent of token blockIdx.x: wave w packs a quarter of its bytes (wave 0 also the
// zero bytes and the scales).
__global__ __launch_bounds__(256) void kv_vpack_kernel(const VPackParams q) {
    const int w = threadIdx.x >> 6;
    vpack_range(q, blockIdx.x, w * q.v_bytes / 4, (w + 1) * q.v_bytes / 4, w == 0, threadIdx.x & 63);
}

// S = the GEMM's K splits (a launch constant): exactly the S partials of each column load.
// CPT columns per thread and pass (2, or 3 for rows wider than 2048 codes: one pass).
template <int DT, int S, int CPT>
__global__ __launch_bounds__(KVS_THR) void kv_store_kernel(const KvStoreParams p) {
    extern __shared__ float s_code[];  // [width]: the token's rounded codes
    const int i = blockIdx.x, tid = threadIdx.x;
    const int64_t slot = load_slot(p.slots, p.slot_bits, i);
    const bool store = slot < p.num_blocks * p.block_size;  // slots past the cache are skipped
    const int64_t row = (slot / p.block_size) * p.c_s0 + (slot % p.block_size) * p.c_s1;
    // Columns c0 + tid + j KVS_THR (j < CPT): every split's partial of each is loaded
    // before the first add (indices clamped, so no branch sits between the loads), then
    // summed in split order.
    for (int c0 = 0; c0 < p.width; c0 += CPT * KVS_THR) {
        float v[CPT][S];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = min(c0 + tid + j * KVS_THR, p.width - 1);
#pragma unroll
            for (int sp = 0; sp < S; ++sp) v[j][sp] = p.part[((int64_t)sp * p.n + i) * p.width + c];
        }
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = c0 + tid + j * KVS_THR;
            float a = v[j][0];
#pragma unroll
            for (int sp = 1; sp < S; ++sp) a += v[j][sp];
            if (c < p.width) {
                const uint16_t r = round_code<DT>(a);
                s_code[c] = code_value<DT>(r);
                if (p.codes && blockIdx.y == 0) p.codes[(int64_t)i * p.co_s0 + c] = r;
                if (!p.quant && store) ((uint16_t*)p.cache)[row + c] = r;
            }
        }
    }
    if (!p.quant || !store) return;
    __syncthreads();
    const int lane = tid & 63;
    uint8_t* dst = (uint8_t*)p.cache + row;
    // Blocks u = y + groups (w + 16 k) of workgroup y, wave w (the H K blocks, then V).
    for (int u = blockIdx.y + p.groups * (tid >> 6); u <= p.H; u += p.groups * (KVS_THR / 64)) {
        if (u < p.H) {
            const float* src = s_code + p.offsets[u];
            pack_k_block([&](int l) { return src[l]; }, p.ranks[u], p.nouts[u], p.offsets[u], u, p.row.ks_off, dst,
                         lane);
        } else {
            const float* src = s_code + p.k_width;
            pack_v_block([&](int c) { return src[c]; }, p.v_rank, p.row.v_nout, p.row.v_nbo, p.row.v_bytes,
                         p.row.vq_off, p.row.vs_off, p.row.nbytes, dst, lane);
        }
    }
}

template <int DT, int CPT>
static const void* kv_store_pick_s(int splits) {
    switch (splits) {
        case 1: return (const void*)&kv_store_kernel<DT, 1, CPT>;
        case 2: return (const void*)&kv_store_kernel<DT, 2, CPT>;
        case 4: return (const void*)&kv_store_kernel<DT, 4, CPT>;
        case 8: return (const void*)&kv_store_kernel<DT, 8, CPT>;
        case 16: return (const void*)&kv_store_kernel<DT, 16, CPT>;
        default: return nullptr;
    }
}
template <int DT>
static const void* kv_store_pick(int splits, int width) {
    return width > 2 * KVS_THR ? kv_store_pick_s<DT, 3>(splits) : kv_store_pick_s<DT, 2>(splits);
}

// K splits: doubled while the GEMM grid has fewer than 256 workgroups (one per CU) and
// every split keeps at least one chunk of K steps.
static int kv_splits(int n, int width, int hidden) {
    const int tiles = ((width + KVW_COLS - 1) / KVW_COLS) * ((n + KVW_TOKENS - 1) / KVW_TOKENS);
    const int ksteps = hidden / 32;
    int s = 1;
    while (s < KVW_MAX_SPLIT && 2 * s * KVW_CHUNK <= ksteps && tiles * s < 256) s *= 2;  // ksteps even
    return s;
}

}  // namespace starkv

using namespace starkv;

extern "C" {

size_t starkv_write_kv_workspace_bytes(int n, int width, int hidden) {
    if (n <= 0 || width <= 0 || hidden < 32) return 0;
    return (size_t)kv_splits(n, width, hidden) * n * width * sizeof(float);
}

}  // extern "C"

namespace starkv {

// One write's launches: the GEMM grid and parameters, then the store's.
struct WriteLaunch {
    hipStream_t stream;
    int w_dtype;
    KvGemmParams g;
    dim3 ggrid;
    KvStoreParams s;
    const void* store_fn;
    size_t lds;
    bool direct;        // the direct form (d, and v for a 3.2-bit row)
    KvDirectParams d;
    VPackParams v;
};

// The calling thread's deferred write (starkv_write_kv_deferred), launched by its next
// decode call on the same stream, by its next write, or by starkv_flush_write.
static thread_local WriteLaunch t_pending;
static thread_local bool t_has_pending = false;

static int prepare_write(WriteLaunch& w, void* stream, const void* hidden, int64_t h_s0, const void* kv_down,
                         int64_t w_s0, int w_dtype, int n, int hidden_size, int k_width, int v_rank, void* cache,
                         int64_t c_s0, int64_t c_s1, int cache_dtype, int block_size, int64_t num_blocks,
                         const void* slot_mapping, int slot_bits, int num_kv_heads, const int32_t* k_ranks,
                         const int32_t* k_offsets, const int32_t* k_nouts, int row_bytes, void* codes_out,
                         int64_t co_s0, void* workspace, size_t workspace_bytes) {
    SKV_CHECK(n >= 0 && k_width > 0 && v_rank > 0 && hidden_size > 0, "write_kv: bad sizes");
    SKV_CHECK(w_dtype == STARKV_BF16 || w_dtype == STARKV_F16, "write_kv: hidden and kv_down must be bf16 or fp16");
    SKV_CHECK(hidden_size % 64 == 0, "write_kv: hidden size %d must be a multiple of 64", hidden_size);
    SKV_CHECK(k_width % 16 == 0, "write_kv: k_width must be a multiple of 16 (head widths are)");
    SKV_CHECK(block_size > 0, "write_kv: block_size must be positive");
    SKV_CHECK(slot_bits == 32 || slot_bits == 64, "write_kv: slot_mapping must be int32 or int64");
    SKV_CHECK(h_s0 >= hidden_size && w_s0 >= hidden_size && h_s0 % 8 == 0 && w_s0 % 8 == 0 &&
                  ((uintptr_t)hidden % 16) == 0 && ((uintptr_t)kv_down % 16) == 0,
              "write_kv: hidden and kv_down rows must be 16-byte aligned and at least hidden_size long");
    const int width = k_width + v_rank;
    const bool quant = row_bytes > 0;
    RowLayout rl{};
    if (quant) {
        SKV_CHECK(num_kv_heads > 0, "write_kv: num_kv_heads must be positive");
        rl = row_layout_host(k_width, num_kv_heads, v_rank);
        SKV_CHECK(row_bytes == rl.nbytes, "write_kv: row_bytes %d != QuantRow.nbytes %d", row_bytes, rl.nbytes);
        SKV_CHECK(c_s0 % 4 == 0 && c_s1 % 4 == 0 && ((uintptr_t)cache % 4) == 0,
                  "write_kv: 3.2-bit cache base and byte strides must be multiples of 4");
        SKV_CHECK(c_s1 >= row_bytes, "write_kv: cache slot stride %lld < row_bytes %d", (long long)c_s1, row_bytes);
    } else {
        SKV_CHECK(cache_dtype == w_dtype, "write_kv: the bf16/fp16 cache must have the model dtype");
        SKV_CHECK(c_s1 >= width, "write_kv: cache slot stride %lld < %d codes", (long long)c_s1, width);
    }
    if (n == 0) return STARKV_OK;
    SKV_CHECK(hidden && kv_down && cache && slot_mapping && workspace, "write_kv: null pointer");
    SKV_CHECK(!quant || (k_ranks && k_offsets && k_nouts), "write_kv: null head arrays");
    SKV_CHECK(!codes_out || co_s0 >= width, "write_kv: codes_out row stride %lld < %d", (long long)co_s0, width);
    const int splits = kv_splits(n, width, hidden_size);
    SKV_CHECK(workspace_bytes >= (size_t)splits * n * width * sizeof(float), "write_kv: workspace %zu bytes < %zu",
              workspace_bytes, (size_t)splits * n * width * sizeof(float));
    SKV_CHECK(((uintptr_t)workspace % 16) == 0, "write_kv: workspace must be 16-byte aligned");

    KvGemmParams g;
    g.hidden = (const uint16_t*)hidden; g.h_s0 = h_s0;
    g.w = (const uint16_t*)kv_down; g.w_s0 = w_s0;
    g.n = n; g.width = width; g.ksteps = hidden_size / 32; g.splits = splits;
    g.part = (float*)workspace;
    const dim3 ggrid((width + KVW_COLS - 1) / KVW_COLS, splits, (n + KVW_TOKENS - 1) / KVW_TOKENS);
    KvStoreParams s;
    s.part = g.part; s.splits = splits; s.n = n; s.width = width;
    s.k_width = k_width; s.v_rank = v_rank;
    s.codes = (uint16_t*)codes_out; s.co_s0 = co_s0;
    s.cache = cache; s.c_s0 = c_s0; s.c_s1 = c_s1;
    s.block_size = block_size; s.num_blocks = num_blocks;
    s.slots = slot_mapping; s.slot_bits = slot_bits;
    s.quant = quant; s.H = num_kv_heads; s.ranks = k_ranks; s.offsets = k_offsets; s.nouts = k_nouts;
    s.row = rl;
    // Few tokens: a token's H + 1 blocks are packed by several workgroups (each one forms
    // the token's codes), one block per wave.
    s.groups = quant && n <= 16 ? std::max(1, std::min(8, (num_kv_heads + 1 + KVS_THR / 64 - 1) / (KVS_THR / 64))) : 1;
    const size_t lds = (size_t)width * sizeof(float);
    SKV_CHECK(lds <= 64 * 1024, "write_kv: %d codes per token exceed the 64 KB LDS block", width);
    // Two tokens only at hidden 4096 (the compiled slice count: registers for both rows).
    w.direct = hidden_size % 512 == 0 && hidden_size <= 512 * KVD_MAX_SLICES &&
               (n == 1 || (n == 2 && hidden_size == 512 * KVD_MAX_SLICES));
    if (w.direct) {
        KvDirectParams& d = w.d;
        memset(&d, 0, sizeof(d));
        d.hidden = (const uint16_t*)hidden; d.h_s0 = h_s0;
        d.w = (const uint16_t*)kv_down; d.w_s0 = w_s0;
        d.n = n; d.slices = hidden_size / 512; d.width = width; d.k_width = k_width; d.v_rank = v_rank;
        d.quant = quant;
        d.codes = (uint16_t*)codes_out; d.co_s0 = co_s0;
        d.cache = cache; d.c_s0 = c_s0; d.c_s1 = c_s1;
        d.block_size = block_size; d.num_blocks = num_blocks;
        d.slots = slot_mapping; d.slot_bits = slot_bits;
        if (quant) {
            // Workspace: the rounded codes [n][width] (uint16), then the V maxima.
            d.k_jobs = num_kv_heads;
            d.kt_jobs = codes_out ? (k_width + 15) / 16 : 0;
            d.vtiles = (v_rank + 15) / 16;
            d.jobs = d.k_jobs + d.kt_jobs + d.vtiles;
            d.ranks = k_ranks; d.offsets = k_offsets; d.nouts = k_nouts; d.ks_off = rl.ks_off;
            d.v_nout = rl.v_nout;
            d.rc = (uint16_t*)workspace;
            const size_t vm_off = ((size_t)n * width * 2 + 15) / 16 * 16;
            d.vmax = (float*)((uint8_t*)workspace + vm_off);
            SKV_CHECK(vm_off + (size_t)n * d.vtiles * 8 <= workspace_bytes, "write_kv: workspace %zu bytes too small",
                      workspace_bytes);
            VPackParams& v = w.v;
            v.rc = d.rc; v.vmax = d.vmax;
            v.n = n; v.width = width; v.k_width = k_width; v.vtiles = d.vtiles; v.dt = w_dtype;
            v.v_rank = v_rank; v.v_nout = rl.v_nout; v.v_nbo = rl.v_nbo; v.v_bytes = rl.v_bytes;
            v.vq_off = rl.vq_off; v.vs_off = rl.vs_off; v.row_bytes = rl.nbytes;
            v.cache = (uint8_t*)cache; v.c_s0 = c_s0; v.c_s1 = c_s1;
            v.block_size = block_size; v.num_blocks = num_blocks;
            v.slots = slot_mapping; v.slot_bits = slot_bits;
        } else {
            d.jobs = (width + 15) / 16;
        }
    }
    w.stream = (hipStream_t)stream;
    w.w_dtype = w_dtype;
    w.g = g;
    w.ggrid = ggrid;
    w.s = s;
    w.store_fn = w_dtype == STARKV_BF16 ? kv_store_pick<STARKV_BF16>(splits, width)
                                        : kv_store_pick<STARKV_F16>(splits, width);
    SKV_CHECK(w.store_fn != nullptr, "write_kv: %d K splits", splits);
    w.lds = lds;
    return STARKV_OK;
}

int launch_vpack_on(const VPackParams& v, hipStream_t stream) {
    hipLaunchKernelGGL(kv_vpack_kernel, dim3(v.n), dim3(256), 0, stream, v);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

// The direct form's V latent (3.2-bit rows; nothing for bf16/fp16 rows).
static int launch_vpack(const WriteLaunch& w) {
    if (!w.d.quant) return STARKV_OK;
    return launch_vpack_on(w.v, w.stream);
}

template <int DT>
static const void* kv_direct_fn(int n, int slices) {
    if (slices == KVD_MAX_SLICES)
        return n == 1 ? (const void*)&kv_direct_kernel<DT, 1, KVD_MAX_SLICES>
                      : (const void*)&kv_direct_kernel<DT, 2, KVD_MAX_SLICES>;
    return (const void*)&kv_direct_kernel<DT, 1, 0>;
}

static int launch_store(WriteLaunch& w) {
    if (w.direct) return launch_vpack(w);
    void* args[] = {(void*)&w.s};
    SKV_HIP(hipLaunchKernel(w.store_fn, dim3(w.s.n, w.s.groups), dim3(KVS_THR), args, w.lds, w.stream));
    return STARKV_OK;
}

static int launch_write(WriteLaunch& w) {
    if (w.direct) {
        const void* fn = w.w_dtype == STARKV_BF16 ? kv_direct_fn<STARKV_BF16>(w.d.n, w.d.slices)
                                                    : kv_direct_fn<STARKV_F16>(w.d.n, w.d.slices);
        void* args[] = {(void*)&w.d};
        SKV_HIP(hipLaunchKernel(fn, dim3(w.d.jobs), dim3(KVW_THR), args, 0, w.stream));
        return launch_vpack(w);
    }
    if (w.w_dtype == STARKV_BF16)
        hipLaunchKernelGGL(kv_gemm_kernel<STARKV_BF16>, w.ggrid, dim3(KVW_THR), 0, w.stream, w.g);
    else
        hipLaunchKernelGGL(kv_gemm_kernel<STARKV_F16>, w.ggrid, dim3(KVW_THR), 0, w.stream, w.g);
    SKV_HIP(hipGetLastError());
    return launch_store(w);
}

bool pending_write_on(hipStream_t stream, PendingGemm* out) {
    if (!t_has_pending || t_pending.stream != stream) return false;
    out->stream = t_pending.stream;
    out->w_dtype = t_pending.w_dtype;
    out->g = t_pending.g;
    out->gx = (int)t_pending.ggrid.x;
    out->gy = (int)t_pending.ggrid.y;
    out->gz = (int)t_pending.ggrid.z;
    out->direct = t_pending.direct;
    out->d = t_pending.d;
    return true;
}

bool take_pending_vpack(VPackParams* out) {
    if (!t_has_pending || !t_pending.direct || !t_pending.d.quant) return false;
    *out = t_pending.v;
    t_has_pending = false;
    return true;
}

int launch_pending_store() {
    if (!t_has_pending) return STARKV_OK;
    t_has_pending = false;
    return launch_store(t_pending);
}

int flush_pending_write() {
    if (!t_has_pending) return STARKV_OK;
    t_has_pending = false;
    return launch_write(t_pending);
}

}  // namespace starkv

extern "C" {

int starkv_write_kv(void* stream, const void* hidden, int64_t h_s0, const void* kv_down, int64_t w_s0, int w_dtype,
                    int n, int hidden_size, int k_width, int v_rank, void* cache, int64_t c_s0, int64_t c_s1,
                    int cache_dtype, int block_size, int64_t num_blocks, const void* slot_mapping, int slot_bits,
                    int num_kv_heads, const int32_t* k_ranks, const int32_t* k_offsets, const int32_t* k_nouts,
                    int row_bytes, void* codes_out, int64_t co_s0, void* workspace, size_t workspace_bytes) {
    clear_error();
    int rc = flush_pending_write();
    if (rc) return rc;
    WriteLaunch w;
    rc = prepare_write(w, stream, hidden, h_s0, kv_down, w_s0, w_dtype, n, hidden_size, k_width, v_rank, cache, c_s0,
                       c_s1, cache_dtype, block_size, num_blocks, slot_mapping, slot_bits, num_kv_heads, k_ranks,
                       k_offsets, k_nouts, row_bytes, codes_out, co_s0, workspace, workspace_bytes);
    if (rc || n == 0) return rc;
    return launch_write(w);
}

int starkv_write_kv_deferred(void* stream, const void* hidden, int64_t h_s0, const void* kv_down, int64_t w_s0,
                             int w_dtype, int n, int hidden_size, int k_width, int v_rank, void* cache, int64_t c_s0,
                             int64_t c_s1, int cache_dtype, int block_size, int64_t num_blocks,
                             const void* slot_mapping, int slot_bits, int num_kv_heads, const int32_t* k_ranks,
                             const int32_t* k_offsets, const int32_t* k_nouts, int row_bytes, void* codes_out,
                             int64_t co_s0, void* workspace, size_t workspace_bytes) {
    clear_error();
    int rc = flush_pending_write();
    if (rc) return rc;
    WriteLaunch w;
    rc = prepare_write(w, stream, hidden, h_s0, kv_down, w_s0, w_dtype, n, hidden_size, k_width, v_rank, cache, c_s0,
                       c_s1, cache_dtype, block_size, num_blocks, slot_mapping, slot_bits, num_kv_heads, k_ranks,
                       k_offsets, k_nouts, row_bytes, codes_out, co_s0, workspace, workspace_bytes);
    if (rc || n == 0) return rc;
    t_pending = w;
    t_has_pending = true;
    return STARKV_OK;
}

int starkv_flush_write(void) {
    clear_error();
    return flush_pending_write();
}

}  // extern "C"
