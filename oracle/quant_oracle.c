/*
 * ORACLE -- test infrastructure only. Nothing in the product links, loads or
 * calls this file; only tests/, the smoke check and bench.py's CPU baseline do,
 * and only as the reference the GPU results are compared with.
 *
 * Plain-C restatement of STAR-KV's 3.2-bit KV quantizer and its paged row
 * format, bit for bit:
 *
 *   _q (the quantizer definition)            kv_quant.py:111-120
 *   n_outlier                                 kv_quant.py:76-77, starkv_serve/kernels/paged_quant.py:46-47
 *   QuantRow byte layout                      starkv_serve/kernels/paged_quant.py:71-111
 *   _pack_k  (per token, per KV head)         starkv_serve/kernels/paged_quant.py:146-172
 *   _pack_v  (per token, head-shared V)       starkv_serve/kernels/paged_quant.py:175-202
 *   slot -> row (slot -1 -> null block 0)     starkv_serve/kernels/paged_quant.py:139-143
 *   unpack_k_ref / unpack_v_ref               kv_quant.py:154-161, 182-188
 *
 * Arithmetic: fp32 IEEE division (correctly rounded, as div_rn / torch's
 * tensor-by-tensor division), rintf in the default round-to-nearest-even mode
 * (libdevice rint / torch.round), clamp, +8. Scales are stored as bfloat16
 * with round-to-nearest-even. Build without -ffast-math.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EPS_F 1e-5f /* fp32(1e-5), the amax floor (paged_quant.py:41) */

int oracle_n_outlier(int rank) { return (int)(0.2 * (double)rank); }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float amax_floor(const float *x, int lo, int hi) {
    float a = 0.0f;
    for (int i = lo; i < hi; ++i) {
        float v = fabsf(x[i]);
        if (v > a) a = v;
    }
    return a < EPS_F ? EPS_F : a;
}

/* code = clamp(rint(x / s), lo, hi) + 8 */
static int qcode(float x, float s, float lo, float hi) {
    volatile float d = x / s; /* one IEEE division, no contraction */
    float q = rintf(d);
    if (q < lo) q = lo;
    if (q > hi) q = hi;
    return (int)(q + 8.0f);
}

/* kv_quant._q over one block: x[n] at `bits` -> codes[n] (0..15) and the fp32 scale. */
void oracle_quantize_block(const float *x, int n, int bits, int *codes, float *scale) {
    float qmax = (float)((1 << (bits - 1)) - 1);
    float qmin = -(float)(1 << (bits - 1));
    volatile float s = amax_floor(x, 0, n) / qmax;
    for (int i = 0; i < n; ++i) codes[i] = qcode(x[i], s, qmin, qmax);
    *scale = s;
}

static void put_bf16(uint8_t *p, float f) {
    uint16_t h = oracle_f32_to_bf16(f);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}

/* One token's K codes (all heads) into row bytes [0, ks_off + 4H). */
void oracle_pack_k_row(const float *x, int num_heads, const int *ranks, const int *offsets,
                       const int *nouts, int ks_off, uint8_t *row) {
    for (int h = 0; h < num_heads; ++h) {
        int R = ranks[h], nout = nouts[h], off = offsets[h];
        int wh = ((R + 15) / 16) * 16; /* stored width; lanes past R are zero codes */
        const float *xh = x + off;
        volatile float s_out = amax_floor(xh, 0, nout) / 7.0f;
        volatile float s_in = amax_floor(xh, nout, wh) / 3.0f;
        for (int k = 0; 2 * k < wh; ++k) {
            int n[2];
            for (int e = 0; e < 2; ++e) {
                int lane = 2 * k + e;
                n[e] = lane < nout ? qcode(xh[lane], s_out, -8.0f, 7.0f)
                                   : qcode(xh[lane], s_in, -4.0f, 3.0f);
            }
            row[off / 2 + k] = (uint8_t)(n[0] | (n[1] << 4));
        }
        put_bf16(row + ks_off + 4 * h, nout > 0 ? s_out : 1.0f);
        put_bf16(row + ks_off + 4 * h + 2, s_in);
    }
}

/* One token's head-shared V codes into row bytes [vs_off, vq_off + v_bytes). */
void oracle_pack_v_row(const float *x, int R, int nout, int vs_off, int vq_off, uint8_t *row) {
    int nbo = (nout + 1) / 2;
    int nb = nbo + (R - nout + 1) / 2;
    volatile float s_out = amax_floor(x, 0, nout) / 7.0f;
    volatile float s_in = amax_floor(x, nout, R) / 3.0f;
    for (int j = 0; j < nb; ++j) {
        int in_out = j < nbo;
        int c_lo = in_out ? 2 * j : nout + 2 * (j - nbo);
        int c_end = in_out ? nout : R;
        float s = in_out ? s_out : s_in;
        float lo = in_out ? -8.0f : -4.0f, hi = in_out ? 7.0f : 3.0f;
        int nl = c_lo < c_end ? qcode(x[c_lo], s, lo, hi) : 8;
        int nh = c_lo + 1 < c_end ? qcode(x[c_lo + 1], s, lo, hi) : 8;
        row[vq_off + j] = (uint8_t)(nl | (nh << 4));
    }
    put_bf16(row + vs_off, nout > 0 ? s_out : 1.0f);
    put_bf16(row + vs_off + 2, s_in);
}

/*
 * pack_kv over n tokens: k[n, W] (row stride k_s0 floats), v[n, R] (v_s0), into the
 * uint8 cache with byte strides c_s0 (block) and c_s1 (slot). slot < 0 -> 0. Returns
 * nonzero (and writes nothing) if a slot lies outside num_blocks * block_size.
 */
int oracle_pack_kv(const float *k, int64_t k_s0, const float *v, int64_t v_s0, int n,
                   uint8_t *cache, int64_t c_s0, int64_t c_s1, int block_size, int64_t num_blocks,
                   const int64_t *slots, int num_heads, const int *ranks, const int *offsets,
                   const int *nouts, int v_rank, int ks_off, int vs_off, int vq_off) {
    int v_nout = oracle_n_outlier(v_rank);
    for (int i = 0; i < n; ++i) { /* refuse slots outside the cache before writing anything */
        int64_t slot = slots[i] < 0 ? 0 : slots[i];
        if (slot >= num_blocks * block_size) return 1;
    }
    for (int i = 0; i < n; ++i) {
        int64_t slot = slots[i] < 0 ? 0 : slots[i];
        uint8_t *row = cache + (slot / block_size) * c_s0 + (slot % block_size) * c_s1;
        oracle_pack_k_row(k + (int64_t)i * k_s0, num_heads, ranks, offsets, nouts, ks_off, row);
        oracle_pack_v_row(v + (int64_t)i * v_s0, v_rank, v_nout, vs_off, vq_off, row);
    }
    return 0;
}

/* Dequantize one row's K lanes [0, k_width) (unpack_k_ref). */
void oracle_unpack_k_row(const uint8_t *row, int num_heads, const int *ranks, const int *offsets,
                         const int *nouts, int ks_off, float *out) {
    for (int h = 0; h < num_heads; ++h) {
        int wh = ((ranks[h] + 15) / 16) * 16, off = offsets[h];
        float so = oracle_bf16_to_f32((uint16_t)(row[ks_off + 4 * h] | (row[ks_off + 4 * h + 1] << 8)));
        float si = oracle_bf16_to_f32((uint16_t)(row[ks_off + 4 * h + 2] | (row[ks_off + 4 * h + 3] << 8)));
        for (int lane = 0; lane < wh; ++lane) {
            int b = row[(off + lane) / 2];
            int nib = ((off + lane) & 1) ? (b >> 4) : (b & 15);
            out[off + lane] = (float)(nib - 8) * (lane < nouts[h] ? so : si);
        }
    }
}

/* Dequantize one row's V channels [0, R) (unpack_v_ref). */
void oracle_unpack_v_row(const uint8_t *row, int R, int nout, int vs_off, int vq_off, float *out) {
    int nbo = (nout + 1) / 2;
    float so = oracle_bf16_to_f32((uint16_t)(row[vs_off] | (row[vs_off + 1] << 8)));
    float si = oracle_bf16_to_f32((uint16_t)(row[vs_off + 2] | (row[vs_off + 3] << 8)));
    for (int c = 0; c < R; ++c) {
        int blk_out = c < nout;
        int idx = blk_out ? c : c - nout;
        int b = row[vq_off + (blk_out ? 0 : nbo) + idx / 2];
        int nib = (idx & 1) ? (b >> 4) : (b & 15);
        out[c] = (float)(nib - 8) * (blk_out ? so : si);
    }
}
