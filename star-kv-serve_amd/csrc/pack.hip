// Cache write path: the bf16/fp16 code scatter and the 3.2-bit quantize + scatter
// (the quantizer and the row packing are in pack_rows.hpp). One wave quantizes one
// (token, KV head) block, or the token's V latent.
#include <stdarg.h>
#include <stdio.h>

#include "kv_gemm.hpp"
#include "pack_rows.hpp"

namespace starkv {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// ---------------------------------------------------------------------------
// bf16/fp16 codes: one workgroup per token copies its K and V codes to the slot.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void write_codes_kernel(const void* __restrict__ k, int64_t k_s0,
                                                          const void* __restrict__ v, int64_t v_s0, int in_dt,
                                                          void* __restrict__ cache, int64_t c_s0, int64_t c_s1,
                                                          int cache_dt, int block_size, int64_t num_blocks,
                                                          const void* __restrict__ slots, int slot_bits,
                                                          int k_width, int v_rank) {
    const int i = blockIdx.x;
    const int64_t slot = load_slot(slots, slot_bits, i);
    if (slot >= num_blocks * block_size) return;
    const int64_t row = (slot / block_size) * c_s0 + (slot % block_size) * c_s1;
    const int width = k_width + v_rank;
    if (in_dt == cache_dt && in_dt != STARKV_F32) {
        const uint16_t* ks = (const uint16_t*)k + (int64_t)i * k_s0;
        const uint16_t* vs = (const uint16_t*)v + (int64_t)i * v_s0;
        uint16_t* dst = (uint16_t*)cache + row;
        for (int c = threadIdx.x; c < width; c += blockDim.x) dst[c] = c < k_width ? ks[c] : vs[c - k_width];
        return;
    }
    for (int c = threadIdx.x; c < width; c += blockDim.x) {
        float x = c < k_width ? load_f(k, (int64_t)i * k_s0 + c, in_dt) : load_f(v, (int64_t)i * v_s0 + c - k_width, in_dt);
        store_f(cache, row + c, cache_dt, x);
    }
}

// ---------------------------------------------------------------------------
// 3.2-bit pack. Grid (n tokens, ceil((H + 1) / 4)); wave u of the token quantizes
// KV head u (u < H) or the V latent (u == H).
// ---------------------------------------------------------------------------
struct PackParams {
    const void* k; int64_t k_s0;
    const void* v; int64_t v_s0;
    int dt;
    uint8_t* cache; int64_t c_s0, c_s1;
    int block_size;
    int64_t num_blocks;
    const void* slots; int slot_bits;
    int H;
    const int32_t* ranks; const int32_t* offsets; const int32_t* nouts;
    int k_width, v_rank, v_nout, v_nbo, v_bytes;
    int ks_off, vs_off, vq_off, row_bytes;
};

__global__ __launch_bounds__(256) void pack_kv_kernel(const PackParams p) {
    const int i = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (u > p.H) return;
    const int64_t slot = load_slot(p.slots, p.slot_bits, i);
    if (slot >= p.num_blocks * p.block_size) return;
    uint8_t* row = p.cache + (slot / p.block_size) * p.c_s0 + (slot % p.block_size) * p.c_s1;

    if (u < p.H) {
        const int64_t base = (int64_t)i * p.k_s0 + p.offsets[u];
        pack_k_block([&](int l) { return load_f(p.k, base + l, p.dt); }, p.ranks[u], p.nouts[u], p.offsets[u], u,
                     p.ks_off, row, lane);
        return;
    }
    const int64_t base = (int64_t)i * p.v_s0;
    pack_v_block([&](int c) { return load_f(p.v, base + c, p.dt); }, p.v_rank, p.v_nout, p.v_nbo, p.v_bytes, p.vq_off,
                 p.vs_off, p.row_bytes, row, lane);
}

}  // namespace starkv

using namespace starkv;

extern "C" {

int starkv_abi_version(void) { return 6; }

const char* starkv_last_error(void) { return g_err; }

int starkv_write_codes(void* stream, const void* k_codes, int64_t k_s0, const void* v_codes, int64_t v_s0,
                       int in_dtype, void* cache, int64_t c_s0, int64_t c_s1, int cache_dtype, int block_size,
                       int64_t num_blocks, const void* slot_mapping, int slot_bits, int n, int k_width,
                       int v_rank) {
    clear_error();
    if (const int rc = flush_pending_write()) return rc;  // a deferred write goes first
    SKV_CHECK(n >= 0 && k_width >= 0 && v_rank >= 0, "write_codes: negative size");
    SKV_CHECK(block_size > 0, "write_codes: block_size must be positive");
    SKV_CHECK(slot_bits == 32 || slot_bits == 64, "write_codes: slot_mapping must be int32 or int64");
    SKV_CHECK(in_dtype >= 0 && in_dtype <= 2 && cache_dtype >= 0 && cache_dtype <= 2, "write_codes: bad dtype");
    if (n == 0) return STARKV_OK;
    SKV_CHECK(k_codes && v_codes && cache && slot_mapping, "write_codes: null pointer");
    hipLaunchKernelGGL(write_codes_kernel, dim3(n), dim3(256), 0, (hipStream_t)stream, k_codes, k_s0, v_codes,
                       v_s0, in_dtype, cache, c_s0, c_s1, cache_dtype, block_size, num_blocks, slot_mapping,
                       slot_bits, k_width, v_rank);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

int starkv_pack_kv(void* stream, const void* k_codes, int64_t k_s0, const void* v_codes, int64_t v_s0,
                   int code_dtype, uint8_t* cache, int64_t c_s0, int64_t c_s1, int block_size, int64_t num_blocks,
                   const void* slot_mapping, int slot_bits, int n, int num_kv_heads, const int32_t* k_ranks,
                   const int32_t* k_offsets, const int32_t* k_nouts, int k_width, int v_rank, int row_bytes) {
    clear_error();
    if (const int rc = flush_pending_write()) return rc;  // a deferred write goes first
    SKV_CHECK(n >= 0 && num_kv_heads > 0 && k_width > 0 && v_rank > 0, "pack_kv: bad sizes");
    SKV_CHECK(k_width % 16 == 0, "pack_kv: k_width must be a multiple of 16 (head widths are)");
    SKV_CHECK(block_size > 0, "pack_kv: block_size must be positive");
    SKV_CHECK(slot_bits == 32 || slot_bits == 64, "pack_kv: slot_mapping must be int32 or int64");
    SKV_CHECK(code_dtype >= 0 && code_dtype <= 2, "pack_kv: bad dtype");
    PackParams p;
    p.k = k_codes; p.k_s0 = k_s0; p.v = v_codes; p.v_s0 = v_s0; p.dt = code_dtype;
    SKV_CHECK(c_s0 % 4 == 0 && c_s1 % 4 == 0 && ((uintptr_t)cache % 4) == 0,
              "pack_kv: cache base and byte strides must be multiples of 4");
    p.cache = cache; p.c_s0 = c_s0; p.c_s1 = c_s1; p.block_size = block_size; p.num_blocks = num_blocks;
    p.slots = slot_mapping; p.slot_bits = slot_bits; p.H = num_kv_heads;
    p.ranks = k_ranks; p.offsets = k_offsets; p.nouts = k_nouts;
    p.k_width = k_width; p.v_rank = v_rank;
    const RowLayout rl = row_layout_host(k_width, num_kv_heads, v_rank);
    p.v_nout = rl.v_nout;
    p.v_nbo = rl.v_nbo;
    p.v_bytes = rl.v_bytes;
    p.ks_off = rl.ks_off;
    p.vs_off = rl.vs_off;
    p.vq_off = rl.vq_off;
    p.row_bytes = rl.nbytes;
    SKV_CHECK(row_bytes == p.row_bytes, "pack_kv: row_bytes %d != QuantRow.nbytes %d", row_bytes, p.row_bytes);
    if (n == 0) return STARKV_OK;
    SKV_CHECK(k_codes && v_codes && cache && slot_mapping && k_ranks && k_offsets && k_nouts, "pack_kv: null pointer");
    hipLaunchKernelGGL(pack_kv_kernel, dim3(n, (num_kv_heads + 1 + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

}  // extern "C"
