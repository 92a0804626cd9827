// 3.2-bit row packing of one (token, KV head) K block or one token's V latent, shared by
// the pack_kv kernel (codes read from memory) and the fused write kernel (codes in LDS).
//
// Quantizer semantics are those of kv_quant._q (kv_quant.py:111-120) as the reference's
// Triton packers apply them (starkv_serve/kernels/paged_quant.py:146-202): amax floored
// at fp32(1e-5), scale = amax / 7 (outliers) or / 3 (inliers) with IEEE division,
// code = clamp(rint(x / scale)) + 8 with round-half-even, scales stored as bfloat16
// (round-to-nearest-even), the outlier scale stored as 1.0 when a block has no outliers.
// Every function is called by one whole wave (the amax is a wave reduction).
#pragma once

#include "common.hpp"

namespace starkv {

// Slot of token i; padding tokens carry -1: the null block (paged_quant.py:141-143).
// Callers skip slots past the cache (num_blocks * block_size) rather than write them.
__device__ __forceinline__ int64_t load_slot(const void* slots, int bits, int i) {
    const int64_t s = bits == 64 ? ((const int64_t*)slots)[i] : (int64_t)((const int32_t*)slots)[i];
    return s < 0 ? 0 : s;
}

__device__ __forceinline__ int quant_code(float x, float s, float lo, float hi) {
    float q = rintf(__fdiv_rn(x, s));
    q = fminf(fmaxf(q, lo), hi);
    return (int)(q + 8.0f);
}

// K block of KV head u: rank R, `nout` outlier lanes, first lane `off` of the row;
// src(l) is the code of the head's lane l, l < align16(R) (lanes past R hold zero codes
// and count as inliers, paged_quant.py:150-163). Nibbles go to row[off / 2 ..], the two
// bf16 scales to row[ks_off + 4 u].
template <class Src>
__device__ __forceinline__ void pack_k_block(Src&& src, int R, int nout, int off, int u, int ks_off, uint8_t* row,
                                             int lane) {
    const int wh = ((R + 15) >> 4) << 4;
    float a_out = 0.f, a_in = 0.f;
    for (int l = lane; l < wh; l += 64) {
        const float x = fabsf(src(l));
        if (l < nout) a_out = fmaxf(a_out, x); else a_in = fmaxf(a_in, x);
    }
    a_out = fmaxf(wave_max(a_out), 1e-5f);
    a_in = fmaxf(wave_max(a_in), 1e-5f);
    const float s_out = __fdiv_rn(a_out, 7.0f);
    const float s_in = __fdiv_rn(a_in, 3.0f);
    for (int kb = lane; 2 * kb < wh; kb += 64) {
        const int l = 2 * kb;
        const int n0 = l < nout ? quant_code(src(l), s_out, -8.f, 7.f) : quant_code(src(l), s_in, -4.f, 3.f);
        const int n1 = l + 1 < nout ? quant_code(src(l + 1), s_out, -8.f, 7.f) : quant_code(src(l + 1), s_in, -4.f, 3.f);
        row[off / 2 + kb] = (uint8_t)(n0 | (n1 << 4));
    }
    if (lane == 0) {
        const uint16_t so = f32_to_bf16_rne(nout > 0 ? s_out : 1.0f), si = f32_to_bf16_rne(s_in);
        *(uint32_t*)(row + ks_off + 4 * u) = (uint32_t)so | ((uint32_t)si << 16);
    }
}

// V latent of rank R: outlier channels [0, nout) at 4 bits, then inliers at 3 bits,
// each block byte-aligned (nbo outlier bytes, nb bytes in all); an odd block ends in a
// padding nibble 8 (paged_quant.py:184-199). src(c) is channel c. Bytes
// [vq_off + nb, row_bytes) are written as zero (the reference leaves them unwritten).
// The pieces (scales from the two maxima, one byte, the tail) are shared with the
// direct write, which packs a row's bytes over several workgroups.
struct VScales {
    float s_out, s_in;
};
// a_out / a_in: max |x| over the outlier / inlier channels (0 when there are none).
__device__ __forceinline__ VScales v_scales(float a_out, float a_in) {
    return VScales{__fdiv_rn(fmaxf(a_out, 1e-5f), 7.0f), __fdiv_rn(fmaxf(a_in, 1e-5f), 3.0f)};
}
template <class Src>
__device__ __forceinline__ uint8_t pack_v_byte(Src&& src, int j, int R, int nout, int nbo, VScales s) {
    const bool in_out = j < nbo;
    const int c_lo = in_out ? 2 * j : nout + 2 * (j - nbo);
    const int c_end = in_out ? nout : R;
    const float sc = in_out ? s.s_out : s.s_in;
    const float lo = in_out ? -8.f : -4.f, hi = in_out ? 7.f : 3.f;
    int nl = 8, nh = 8;
    if (c_lo < c_end) nl = quant_code(src(c_lo), sc, lo, hi);
    if (c_lo + 1 < c_end) nh = quant_code(src(c_lo + 1), sc, lo, hi);
    return (uint8_t)(nl | (nh << 4));
}
// The zero bytes after the codes (lanes of one wave) and the two scales (lane 0).
__device__ __forceinline__ void pack_v_tail(VScales s, int nout, int nb, int vq_off, int vs_off, int row_bytes,
                                            uint8_t* row, int lane) {
    for (int j = vq_off + nb + lane; j < row_bytes; j += 64) row[j] = 0;
    if (lane == 0) {
        const uint16_t so = f32_to_bf16_rne(nout > 0 ? s.s_out : 1.0f), si = f32_to_bf16_rne(s.s_in);
        *(uint32_t*)(row + vs_off) = (uint32_t)so | ((uint32_t)si << 16);
    }
}

template <class Src>
__device__ __forceinline__ void pack_v_block(Src&& src, int R, int nout, int nbo, int nb, int vq_off, int vs_off,
                                             int row_bytes, uint8_t* row, int lane) {
    float a_out = 0.f, a_in = 0.f;
    for (int c = lane; c < R; c += 64) {
        const float x = fabsf(src(c));
        if (c < nout) a_out = fmaxf(a_out, x); else a_in = fmaxf(a_in, x);
    }
    const VScales s = v_scales(wave_max(a_out), wave_max(a_in));
    for (int j = lane; j < nb; j += 64) row[vq_off + j] = pack_v_byte(src, j, R, nout, nbo, s);
    pack_v_tail(s, nout, nb, vq_off, vs_off, row_bytes, row, lane);
}

__device__ __forceinline__ float code_value_rt(uint16_t r, int dt) {
    return dt == STARKV_BF16 ? bf16_bits_to_f32(r) : (float)__builtin_bit_cast(_Float16, r);
}

// The V latent's bytes [j0, j1) of token t from rounded codes rc [n][width] (model dtype
// dt; V codes from column k_width) and the maxima of their 16-code groups per class,
// vmax [n][vtiles] (outlier, inlier): the direct write's workspace. One wave; `tail`:
// also the zero bytes and the two scales. The maxima of the groups are the block's, so
// the bytes are pack_v_block's.
struct VPackParams {
    const uint16_t* rc; const float* vmax;
    int n, width, k_width, vtiles, dt;
    int v_rank, v_nout, v_nbo, v_bytes, vq_off, vs_off, row_bytes;
    uint8_t* cache; int64_t c_s0, c_s1;
    int block_size; int64_t num_blocks;
    const void* slots; int slot_bits;
};

__device__ __forceinline__ void vpack_range(const VPackParams& q, int t, int j0, int j1, bool tail, int lane) {
    const int64_t slot = load_slot(q.slots, q.slot_bits, t);
    if (slot >= q.num_blocks * q.block_size) return;  // past the cache: skipped
    uint8_t* row = q.cache + (slot / q.block_size) * q.c_s0 + (slot % q.block_size) * q.c_s1;
    const float2* vm = (const float2*)q.vmax + (int64_t)t * q.vtiles;
    float a_out = 0.f, a_in = 0.f;
    for (int i = lane; i < q.vtiles; i += 64) {
        const float2 m = vm[i];
        a_out = fmaxf(a_out, m.x);
        a_in = fmaxf(a_in, m.y);
    }
    const VScales s = v_scales(wave_max(a_out), wave_max(a_in));
    const uint16_t* src = q.rc + (int64_t)t * q.width + q.k_width;
    const int dt = q.dt;
    for (int j = j0 + lane; j < j1; j += 64)
        row[q.vq_off + j] = pack_v_byte([&](int c) { return code_value_rt(src[c], dt); }, j, q.v_rank, q.v_nout,
                                        q.v_nbo, s);
    if (tail) pack_v_tail(s, q.v_nout, q.v_bytes, q.vq_off, q.vs_off, q.row_bytes, row, lane);
}

// vpack_range in two steps for a range of at most 64 bytes and at most 128 maxima per
// token (tokens < 2): vpack_load issues the loads (the lane's maxima, the codes of its
// byte, the slot), vpack_store forms and stores the bytes, so work can sit between the
// loads and their use.
struct VPackPre {
    float mo[2], mi[2];
    uint16_t lo[2], hi[2];
    int64_t slot[2];
};
__device__ __forceinline__ bool vpack_two_step(const VPackParams& q, int j0, int j1) {
    return q.n <= 2 && q.vtiles <= 128 && j1 - j0 <= 64;
}
__device__ __forceinline__ int vpack_lo_channel(const VPackParams& q, int j) {
    return j < q.v_nbo ? 2 * j : q.v_nout + 2 * (j - q.v_nbo);
}
__device__ __forceinline__ VPackPre vpack_load(const VPackParams& q, int j0, int j1, int lane) {
    VPackPre r;
    const int j = min(j0 + lane, max(j1 - 1, 0));
    const int c = min(vpack_lo_channel(q, j), q.v_rank - 1), c1 = min(c + 1, q.v_rank - 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int tt = min(t, q.n - 1);
        r.slot[t] = load_slot(q.slots, q.slot_bits, tt);
        const float2* vm = (const float2*)q.vmax + (int64_t)tt * q.vtiles;
        const float2 a = vm[min(lane, q.vtiles - 1)], b = vm[min(lane + 64, q.vtiles - 1)];
        r.mo[t] = fmaxf(a.x, b.x);
        r.mi[t] = fmaxf(a.y, b.y);
        const uint16_t* src = q.rc + (int64_t)tt * q.width + q.k_width;
        r.lo[t] = src[c];
        r.hi[t] = src[c1];
    }
    return r;
}
__device__ __forceinline__ void vpack_store(const VPackParams& q, const VPackPre& r, int j0, int j1, bool tail,
                                            int lane) {
    const int j = j0 + lane, c = vpack_lo_channel(q, min(j, max(j1 - 1, 0)));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        if (t >= q.n) break;
        const VScales s = v_scales(wave_max(r.mo[t]), wave_max(r.mi[t]));
        if (r.slot[t] >= q.num_blocks * q.block_size) continue;  // past the cache: skipped
        uint8_t* row = q.cache + (r.slot[t] / q.block_size) * q.c_s0 + (r.slot[t] % q.block_size) * q.c_s1;
        const float vlo = code_value_rt(r.lo[t], q.dt), vhi = code_value_rt(r.hi[t], q.dt);
        if (j < j1)
            row[q.vq_off + j] = pack_v_byte([&](int ch) { return ch == c ? vlo : vhi; }, j, q.v_rank, q.v_nout,
                                            q.v_nbo, s);
        if (tail) pack_v_tail(s, q.v_nout, q.v_bytes, q.vq_off, q.vs_off, q.row_bytes, row, lane);
    }
}

// QuantRow (paged_quant.py:71-111) on the host: V outlier channels, V outlier bytes,
// V bytes, K-scale / V-scale / V-code offsets and the row size (16-byte aligned).
struct RowLayout {
    int v_nout, v_nbo, v_bytes, ks_off, vs_off, vq_off, nbytes;
};
static inline int n_outlier_host(int rank) { return (int)(0.2 * (double)rank); }
static inline RowLayout row_layout_host(int k_width, int num_kv_heads, int v_rank) {
    RowLayout r;
    r.v_nout = n_outlier_host(v_rank);
    r.v_nbo = (r.v_nout + 1) / 2;
    r.v_bytes = r.v_nbo + (v_rank - r.v_nout + 1) / 2;
    r.ks_off = k_width / 2;
    r.vs_off = r.ks_off + 4 * num_kv_heads;
    r.vq_off = r.vs_off + 4;
    r.nbytes = (r.vq_off + r.v_bytes + 15) / 16 * 16;
    return r;
}

}  // namespace starkv
