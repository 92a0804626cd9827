// Cache write path: the bf16/fp16 code scatter and the 3.2-bit quantize + scatter.
//
// Quantizer semantics are those of kv_quant._q (kv_quant.py:111-120) as the
// reference's Triton packers apply them (starkv_serve/kernels/paged_quant.py:146-202):
// amax floored at fp32(1e-5), scale = amax / 7 (outliers) or / 3 (inliers) with IEEE
// division, code = clamp(rint(x / scale)) + 8 with round-half-even, scales stored as
// bfloat16 (round-to-nearest-even), the outlier scale stored as 1.0 when a block has
// no outliers. One wave quantizes one (token, KV head) block, or the token's V latent.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace starkv {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

__device__ __forceinline__ int64_t load_slot(const void* slots, int bits, int i) {
    int64_t s = bits == 64 ? ((const int64_t*)slots)[i] : (int64_t)((const int32_t*)slots)[i];
    return s < 0 ? 0 : s;  // padding tokens carry -1: the null block (paged_quant.py:141-143)
}

// Slots past the cache (num_blocks * block_size) are skipped rather than written.

__device__ __forceinline__ int quant_code(float x, float s, float lo, float hi) {
    float q = rintf(__fdiv_rn(x, s));
    q = fminf(fmaxf(q, lo), hi);
    return (int)(q + 8.0f);
}

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
        const int R = p.ranks[u], nout = p.nouts[u], off = p.offsets[u];
        const int wh = ((R + 15) >> 4) << 4;  // stored width: lanes past R hold zero codes
        const int64_t base = (int64_t)i * p.k_s0 + off;
        float a_out = 0.f, a_in = 0.f;
        for (int l = lane; l < wh; l += 64) {
            float x = fabsf(load_f(p.k, base + l, p.dt));
            if (l < nout) a_out = fmaxf(a_out, x); else a_in = fmaxf(a_in, x);
        }
        a_out = fmaxf(wave_max(a_out), 1e-5f);
        a_in = fmaxf(wave_max(a_in), 1e-5f);
        const float s_out = __fdiv_rn(a_out, 7.0f);
        const float s_in = __fdiv_rn(a_in, 3.0f);
        for (int kb = lane; 2 * kb < wh; kb += 64) {
            int n0, n1;
            {
                int l = 2 * kb;
                float x = load_f(p.k, base + l, p.dt);
                n0 = l < nout ? quant_code(x, s_out, -8.f, 7.f) : quant_code(x, s_in, -4.f, 3.f);
                x = load_f(p.k, base + l + 1, p.dt);
                n1 = l + 1 < nout ? quant_code(x, s_out, -8.f, 7.f) : quant_code(x, s_in, -4.f, 3.f);
            }
            row[off / 2 + kb] = (uint8_t)(n0 | (n1 << 4));
        }
        if (lane == 0) {
            uint16_t so = f32_to_bf16_rne(nout > 0 ? s_out : 1.0f), si = f32_to_bf16_rne(s_in);
            *(uint32_t*)(row + p.ks_off + 4 * u) = (uint32_t)so | ((uint32_t)si << 16);
        }
        return;
    }

    // V latent: outlier channels [0, nout) at 4 bits, then inliers at 3 bits, each
    // block byte-aligned; an odd block ends in a padding nibble 8 (paged_quant.py:184-199).
    const int R = p.v_rank, nout = p.v_nout, nbo = p.v_nbo, nb = p.v_bytes;
    const int64_t base = (int64_t)i * p.v_s0;
    float a_out = 0.f, a_in = 0.f;
    for (int c = lane; c < R; c += 64) {
        float x = fabsf(load_f(p.v, base + c, p.dt));
        if (c < nout) a_out = fmaxf(a_out, x); else a_in = fmaxf(a_in, x);
    }
    a_out = fmaxf(wave_max(a_out), 1e-5f);
    a_in = fmaxf(wave_max(a_in), 1e-5f);
    const float s_out = __fdiv_rn(a_out, 7.0f);
    const float s_in = __fdiv_rn(a_in, 3.0f);
    for (int j = lane; j < nb; j += 64) {
        const bool in_out = j < nbo;
        const int c_lo = in_out ? 2 * j : nout + 2 * (j - nbo);
        const int c_end = in_out ? nout : R;
        const float s = in_out ? s_out : s_in;
        const float lo = in_out ? -8.f : -4.f, hi = in_out ? 7.f : 3.f;
        int nl = 8, nh = 8;
        if (c_lo < c_end) nl = quant_code(load_f(p.v, base + c_lo, p.dt), s, lo, hi);
        if (c_lo + 1 < c_end) nh = quant_code(load_f(p.v, base + c_lo + 1, p.dt), s, lo, hi);
        row[p.vq_off + j] = (uint8_t)(nl | (nh << 4));
    }
    // The row's trailing pad bytes are defined here as zero.
    for (int j = p.vq_off + nb + lane; j < p.row_bytes; j += 64) row[j] = 0;
    if (lane == 0) {
        uint16_t so = f32_to_bf16_rne(nout > 0 ? s_out : 1.0f), si = f32_to_bf16_rne(s_in);
        *(uint32_t*)(row + p.vs_off) = (uint32_t)so | ((uint32_t)si << 16);
    }
}

static int n_outlier_host(int rank) { return (int)(0.2 * (double)rank); }

}  // namespace starkv

using namespace starkv;

extern "C" {

int starkv_abi_version(void) { return 1; }

const char* starkv_last_error(void) { return g_err; }

int starkv_write_codes(void* stream, const void* k_codes, int64_t k_s0, const void* v_codes, int64_t v_s0,
                       int in_dtype, void* cache, int64_t c_s0, int64_t c_s1, int cache_dtype, int block_size,
                       int64_t num_blocks, const void* slot_mapping, int slot_bits, int n, int k_width,
                       int v_rank) {
    clear_error();
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
    p.v_nout = n_outlier_host(v_rank);
    p.v_nbo = (p.v_nout + 1) / 2;
    p.v_bytes = p.v_nbo + (v_rank - p.v_nout + 1) / 2;
    p.ks_off = k_width / 2;
    p.vs_off = p.ks_off + 4 * num_kv_heads;
    p.vq_off = p.vs_off + 4;
    p.row_bytes = (p.vq_off + p.v_bytes + 15) / 16 * 16;
    SKV_CHECK(row_bytes == p.row_bytes, "pack_kv: row_bytes %d != QuantRow.nbytes %d", row_bytes, p.row_bytes);
    if (n == 0) return STARKV_OK;
    SKV_CHECK(k_codes && v_codes && cache && slot_mapping && k_ranks && k_offsets && k_nouts, "pack_kv: null pointer");
    hipLaunchKernelGGL(pack_kv_kernel, dim3(n, (num_kv_heads + 1 + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

}  // extern "C"
