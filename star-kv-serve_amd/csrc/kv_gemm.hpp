// The code GEMM of the fused cache write, shared by the write launch (kv_write.hip) and
// by the decode's first launch when a deferred write rides in it (decode.hip), and the
// deferred-write state. Two forms: split-K partial products on MFMA (any token count;
// a store launch sums them), and for one or two tokens the direct form, whose
// workgroups own whole codes and store them (or pack the 3.2-bit K blocks) themselves.
//
// Reference: the model's code GEMM (starkv_serve/model.py:71: kv = F.linear(hidden,
// kv_down), kv_down = [k_down; v_down], attention.py:161).
#pragma once

#include "common.hpp"
#include "pack_rows.hpp"

namespace starkv {

constexpr int KVW_THR = 256;    // GEMM workgroup
constexpr int KVW_COLS = 64;    // codes per GEMM workgroup (4 waves x 16)
constexpr int KVW_TOKENS = 64;  // tokens per GEMM workgroup (4 MFMA row tiles)
constexpr int KVW_MAX_SPLIT = 16;
constexpr int KVW_CHUNK = 8;     // K steps (of 32 channels) whose loads are in flight together

struct KvGemmParams {
    const uint16_t* hidden; int64_t h_s0;  // [n, hidden] elements
    const uint16_t* w; int64_t w_s0;       // kv_down [width, hidden]
    int n, width, ksteps, splits;           // ksteps = hidden / 32
    float* part;                            // [splits][n][width]
};

template <int DT>
__device__ __forceinline__ f32x4_t mfma_16x16x32(uint4 a, uint4 b, f32x4_t c) {
    if constexpr (DT == STARKV_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                      0, 0, 0);
}

// K steps [k0, k1) of one wave: TILES row tiles (uniform per workgroup) x 16 codes.
// The channel sum is order-free, so the channels go to MFMA steps in an order that
// reads whole lines: over steps 2m and 2m + 1, lane group g (lane / 16) supplies
// channels 64 m + 16 g .. + 8 and then + 8 .. + 16 of its row, 32 contiguous bytes,
// and the 4 groups cover the row's 128 bytes; A (hidden) and B (kv_down) use the same
// order. Every load of a chunk of KVW_CHUNK steps is issued before its first MFMA; pairs
// past the split's end reload its last pair with B zeroed (no branch between loads).
template <int DT, int TILES>
__device__ __forceinline__ void kv_gemm_steps(const uint16_t* wr, const uint16_t* const (&ar)[4], int k0, int k1,
                                              f32x4_t (&acc)[4]) {
    for (int kc = k0; kc < k1; kc += KVW_CHUNK) {
        uint4 b[KVW_CHUNK], a[KVW_CHUNK][TILES];
#pragma unroll
        for (int j = 0; j < KVW_CHUNK; j += 2) {
            const int m = min(kc + j, k1 - 2) >> 1;  // the pair's 64-channel block
            b[j] = *(const uint4*)(wr + 64 * m);
            b[j + 1] = *(const uint4*)(wr + 64 * m + 8);
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                a[j][t] = *(const uint4*)(ar[t] + 64 * m);
                a[j + 1][t] = *(const uint4*)(ar[t] + 64 * m + 8);
            }
        }
#pragma unroll
        for (int j = 0; j < KVW_CHUNK; ++j) {
            const uint4 bj = kc + j < k1 ? b[j] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TILES; ++t) acc[t] = mfma_16x16x32<DT>(a[j][t], bj, acc[t]);
        }
    }
}

// Workgroup (bx, by, bz) of the GEMM grid (code tile, K split, token block); KVW_THR
// threads.
template <int DT>
__device__ __forceinline__ void kv_gemm_block(const KvGemmParams& p, int bx, int by, int bz) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int s = by, m0 = KVW_TOKENS * bz;
    const int col = KVW_COLS * bx + 16 * wave + (lane & 15);  // this lane's B column (code)
    const int kq = 16 * (lane >> 4);                                   // its 16 channels of each 64
    // Splits cover whole pairs of K steps (ksteps is even: hidden is a multiple of 64).
    const int k0 = 2 * (s * (p.ksteps / 2) / p.splits), k1 = 2 * ((s + 1) * (p.ksteps / 2) / p.splits);
    const int tiles = min(4, (p.n - m0 + 15) / 16);  // row tiles with tokens (uniform)
    // Rows past the code or token range read row width - 1 / n - 1 (valid memory);
    // their products are never stored.
    const uint16_t* wr = p.w + (int64_t)min(col, p.width - 1) * p.w_s0 + kq;
    const uint16_t* ar[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) ar[t] = p.hidden + (int64_t)min(m0 + 16 * t + (lane & 15), p.n - 1) * p.h_s0 + kq;
    f32x4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    switch (tiles) {
        case 1: kv_gemm_steps<DT, 1>(wr, ar, k0, k1, acc); break;
        case 2: kv_gemm_steps<DT, 2>(wr, ar, k0, k1, acc); break;
        case 3: kv_gemm_steps<DT, 3>(wr, ar, k0, k1, acc); break;
        default: kv_gemm_steps<DT, 4>(wr, ar, k0, k1, acc); break;
    }
    if (col >= p.width) return;
    // acc[t][e] = code `col` of token m0 + 16 t + 4 (lane >> 4) + e.
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = m0 + 16 * t + 4 * (lane >> 4) + e;
            if (t < tiles && m < p.n) p.part[((int64_t)s * p.n + m) * p.width + col] = acc[t][e];
        }
}


template <int DT>
__device__ __forceinline__ uint16_t round_code(float x) {
    if constexpr (DT == STARKV_BF16) return f32_to_bf16_rne(x);
    else return __builtin_bit_cast(uint16_t, (_Float16)x);
}
template <int DT>
__device__ __forceinline__ float code_value(uint16_t r) {
    if constexpr (DT == STARKV_BF16) return bf16_bits_to_f32(r);
    else return (float)__builtin_bit_cast(_Float16, r);
}

// ---------------------------------------------------------------------------
// The direct write: one token with hidden a multiple of 512 up to 512 KVD_MAX_SLICES, or
// KVD_MAX_TOKENS tokens with hidden 512 KVD_MAX_SLICES. Job j of a launch owns whole
// codes: 16 codes (the bf16/fp16 row's codes, a 3.2-bit row's V codes, or K codes asked
// for as codes_out only), or the K block of KV head j (3.2-bit), which it packs itself. Lane l of a wave holds channels
// 512 s + 8 l .. + 8 (s < slices) of each token row and of KVD_COLS kv_down rows, and a
// code is the wave sum of the lanes' fp32 dot products (a fixed order). The V latent of
// a 3.2-bit row needs its maxima over all V codes: V jobs store the rounded codes and
// their 16-code maxima (per outlier / inlier class) in the workspace, and vpack_range
// packs the bytes afterwards (its own launch, or the next decode's logits pass).
// ---------------------------------------------------------------------------
constexpr int KVD_MAX_TOKENS = 2;
constexpr int KVD_MAX_SLICES = 8;   // hidden <= 4096
constexpr int KVD_COLS = 4;         // codes per wave and round (16 per workgroup)
constexpr int KVD_KB = 128;         // K blocks up to this width are packed from LDS

struct KvDirectParams {
    const uint16_t* hidden; int64_t h_s0;
    const uint16_t* w; int64_t w_s0;
    int n, slices, width, k_width, v_rank;
    int quant, k_jobs, kt_jobs, jobs;    // 3.2-bit: K block jobs (num_kv_heads), K code-only jobs
    uint16_t* codes; int64_t co_s0;      // optional [n, width] rounded codes
    void* cache; int64_t c_s0, c_s1;     // element strides (bytes for the 3.2-bit cache)
    int block_size; int64_t num_blocks;
    const void* slots; int slot_bits;
    const int32_t* ranks; const int32_t* offsets; const int32_t* nouts; int ks_off;
    int v_nout;
    uint16_t* rc;                        // 3.2-bit: [n][width] rounded codes (V, wide K blocks)
    float* vmax;                         // 3.2-bit: [n][vtiles][2] max |code| of 16 V codes per class
    int vtiles;
};

// acc += the fp32 products of 8 bf16/fp16 channels of a kv_down row (w) and a token row (h).
template <int DT>
__device__ __forceinline__ void kvd_dot8(uint4 w, uint4 h, float& acc) {
    const uint32_t wa[4] = {w.x, w.y, w.z, w.w}, ha[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (DT == STARKV_BF16) {
            acc = fmaf(__uint_as_float(wa[e] << 16), __uint_as_float(ha[e] << 16), acc);
            acc = fmaf(__uint_as_float(wa[e] & 0xffff0000u), __uint_as_float(ha[e] & 0xffff0000u), acc);
        } else {
            acc = fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)wa[e]),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)ha[e]), acc);
            acc = fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(wa[e] >> 16)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(ha[e] >> 16)), acc);
        }
    }
}

// Job `job` of the direct write; a workgroup of 256 threads (4 waves). SL: the slices
// (hidden / 512) when known at compile time (hidden 4096), else 0 (p.slices, guarded).
// Each round's kv_down loads are issued first, then the token rows', and the slots are
// read only for the stores, so the rows' latency is the only one before the products.
template <int DT, int TOK, int SL>
__device__ __forceinline__ void kv_direct_block(const KvDirectParams& p, int job) {
    __shared__ float s_k[TOK][KVD_KB];
    __shared__ float s_vm[4][TOK][2];
    constexpr int NS = SL > 0 ? SL : KVD_MAX_SLICES;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // kind 0: bf16/fp16 row codes; 1: K block of head u; 2: K codes for codes_out only; 3: V codes
    int c0, nc, kind, u = 0;
    if (!p.quant) {
        c0 = 16 * job; nc = min(16, p.width - c0); kind = 0;
    } else if (job < p.k_jobs) {
        u = job; c0 = p.offsets[u]; nc = ((p.ranks[u] + 15) >> 4) << 4; kind = 1;
    } else if (job < p.k_jobs + p.kt_jobs) {
        c0 = 16 * (job - p.k_jobs); nc = min(16, p.k_width - c0); kind = 2;
    } else {
        c0 = p.k_width + 16 * (job - p.k_jobs - p.kt_jobs); nc = min(16, p.width - c0); kind = 3;
    }
    const int S = SL > 0 ? SL : p.slices;
    // Lane i TOK + t (< KVD_COLS TOK) stores code cb + i of token t.
    const int li = lane / TOK, lt = lane % TOK;
    const bool lane_st = lane < KVD_COLS * TOK && lt < p.n;
    float vmo = 0.f, vmi = 0.f;  // kind 3: this lane's |code| by class
    uint4 hv[TOK][NS];
    // The products of round cb (this wave's KVD_COLS codes from cb) are summed over the
    // wave and stored.
    auto finish = [&](int cb, float (&acc)[KVD_COLS][TOK]) {
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < KVD_COLS; ++i)
#pragma unroll
            for (int t = 0; t < TOK; ++t) {
                const float a = wave_sum(acc[i][t]);
                if (lane == i * TOK + t) v = a;
            }
        const int c = cb + li;
        if (!lane_st || c >= c0 + nc) return;
        const uint16_t r = round_code<DT>(v);
        if (p.codes && kind != 1) p.codes[(int64_t)lt * p.co_s0 + c] = r;
        if (kind == 0) {
            const int64_t slot = load_slot(p.slots, p.slot_bits, lt);
            if (slot < p.num_blocks * p.block_size)
                ((uint16_t*)p.cache)[(slot / p.block_size) * p.c_s0 + (slot % p.block_size) * p.c_s1 + c] = r;
        } else if (kind == 1) {
            if (nc <= KVD_KB) s_k[lt][c - c0] = code_value<DT>(r);
            else p.rc[(int64_t)lt * p.width + c] = r;
        } else if (kind == 3) {
            p.rc[(int64_t)lt * p.width + c] = r;
            const float x = fabsf(code_value<DT>(r));
            if (c - p.k_width < p.v_nout) vmo = x; else vmi = x;
        }
    };
    auto load_w = [&](uint4 (&wv)[KVD_COLS][NS], int cb, int s) {
#pragma unroll
        for (int i = 0; i < KVD_COLS; ++i)
            wv[i][s] = *(const uint4*)(p.w + (int64_t)min(cb + i, p.width - 1) * p.w_s0 + 512 * min(s, S - 1) +
                                       8 * lane);
    };
    auto load_h = [&]() {
#pragma unroll
        for (int t = 0; t < TOK; ++t)
#pragma unroll
            for (int s = 0; s < NS; ++s)
                hv[t][s] = *(const uint4*)(p.hidden + (int64_t)min(t, p.n - 1) * p.h_s0 + 512 * min(s, S - 1) + 8 * lane);
    };
    auto dot = [&](const uint4 (&wv)[KVD_COLS][NS], int s, float (&acc)[KVD_COLS][TOK]) {
        if (SL > 0 || s < S) {
#pragma unroll
            for (int i = 0; i < KVD_COLS; ++i)
#pragma unroll
                for (int t = 0; t < TOK; ++t) kvd_dot8<DT>(wv[i][s], hv[t][s], acc[i][t]);
        }
    };
    if (SL > 0 && nc == 32) {
        // Two rounds (a K block of 17 .. 32 codes), straight-line: as slice s of the first
        // round is used, its registers take slice s of the second, so the block's kv_down
        // rows stream with one round trip.
        uint4 wv[KVD_COLS][NS];
        float a0[KVD_COLS][TOK], a1[KVD_COLS][TOK];
#pragma unroll
        for (int s = 0; s < NS; ++s) load_w(wv, c0 + KVD_COLS * wave, s);
        load_h();
#pragma unroll
        for (int i = 0; i < KVD_COLS; ++i)
#pragma unroll
            for (int t = 0; t < TOK; ++t) a0[i][t] = a1[i][t] = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            dot(wv, s, a0);
            load_w(wv, c0 + 16 + KVD_COLS * wave, s);
            __builtin_amdgcn_sched_barrier(0);  // the reload stays here (not sunk past later products)
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) dot(wv, s, a1);
        finish(c0 + KVD_COLS * wave, a0);
        finish(c0 + 16 + KVD_COLS * wave, a1);
    } else {
        for (int cr = c0; cr < c0 + nc; cr += 16) {
            const int cb = cr + KVD_COLS * wave;
            uint4 wv[KVD_COLS][NS];
#pragma unroll
            for (int s = 0; s < NS; ++s) load_w(wv, cb, s);
            if (cr == c0) load_h();
            float acc[KVD_COLS][TOK];
#pragma unroll
            for (int i = 0; i < KVD_COLS; ++i)
#pragma unroll
                for (int t = 0; t < TOK; ++t) acc[i][t] = 0.f;
#pragma unroll
            for (int s = 0; s < NS; ++s) dot(wv, s, acc);
            finish(cb, acc);
        }
    }
    if (kind == 1) {
        __syncthreads();
        if (wave < p.n) {
            const int64_t sl = load_slot(p.slots, p.slot_bits, wave);
            if (sl < p.num_blocks * p.block_size) {
                uint8_t* row = (uint8_t*)p.cache + (sl / p.block_size) * p.c_s0 + (sl % p.block_size) * p.c_s1;
                const uint16_t* rw = p.rc + (int64_t)wave * p.width + c0;
                const float* sk = &s_k[wave < TOK ? wave : 0][0];
                const bool lds = nc <= KVD_KB;
                pack_k_block([&](int l) { return lds ? sk[l] : code_value<DT>(rw[l]); }, p.ranks[u], p.nouts[u], c0, u,
                             p.ks_off, row, lane);
            }
        }
    } else if (kind == 3) {
        // The job's 16-code maxima per token and class.
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            const float mo = wave_max(lt == t && lane_st ? vmo : 0.f);
            const float mi = wave_max(lt == t && lane_st ? vmi : 0.f);
            if (lane == 0) {
                s_vm[wave][t][0] = mo;
                s_vm[wave][t][1] = mi;
            }
        }
        __syncthreads();
        if (threadIdx.x < 2 * TOK && (int)threadIdx.x / 2 < p.n) {
            const int t = threadIdx.x / 2, k = threadIdx.x & 1;
            const float m = fmaxf(fmaxf(s_vm[0][t][k], s_vm[1][t][k]), fmaxf(s_vm[2][t][k], s_vm[3][t][k]));
            p.vmax[((int64_t)t * p.vtiles + (job - p.k_jobs - p.kt_jobs)) * 2 + k] = m;
        }
    }
}

// A write recorded by starkv_write_kv_deferred and not launched yet (one per host
// thread): its GEMM grid and parameters; the store is launched by kv_write.hip.
struct PendingGemm {
    hipStream_t stream;
    int w_dtype;
    KvGemmParams g;
    int gx, gy, gz;  // GEMM grid (code tiles, K splits, token blocks)
    bool direct;     // the direct form instead: d.jobs workgroups
    KvDirectParams d;
};

// The calling thread's pending write, if it is on `stream` (the caller then launches its
// GEMM workgroups and calls launch_pending_store).
bool pending_write_on(hipStream_t stream, PendingGemm* out);
// A direct 3.2-bit pending write whose GEMM has been launched: its V latents' parameters,
// for the decode's logits pass to pack; the write is then done (no longer pending).
bool take_pending_vpack(VPackParams* out);
// Launches the V latents of a direct 3.2-bit write (kv_vpack_kernel).
int launch_vpack_on(const VPackParams& v, hipStream_t stream);
// Launches the pending write's store after its GEMM (the split form's store, the direct
// form's V latent for a 3.2-bit row, nothing for a direct bf16/fp16 row) and clears it.
int launch_pending_store();
// Launches the calling thread's pending write (GEMM, then store) on its own stream and
// clears it; nothing when none is pending.
int flush_pending_write();

}  // namespace starkv
