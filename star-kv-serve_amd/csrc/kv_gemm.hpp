// The code GEMM of the fused cache write (codes = hidden @ kv_down^T as split-K partial
// products on MFMA), shared by the write launch (kv_write.hip) and by the decode's first
// launch when a deferred write rides in it (decode.hip), and the deferred-write state.
//
// Reference: the model's code GEMM (starkv_serve/model.py:71: kv = F.linear(hidden,
// kv_down), kv_down = [k_down; v_down], attention.py:161).
#pragma once

#include "common.hpp"

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


// A write recorded by starkv_write_kv_deferred and not launched yet (one per host
// thread): its GEMM grid and parameters; the store is launched by kv_write.hip.
struct PendingGemm {
    hipStream_t stream;
    int w_dtype;
    KvGemmParams g;
    int gx, gy, gz;  // GEMM grid (code tiles, K splits, token blocks)
};

// The calling thread's pending write, if it is on `stream` (the caller then launches its
// GEMM workgroups and calls launch_pending_store).
bool pending_write_on(hipStream_t stream, PendingGemm* out);
// Launches the pending write's store after its GEMM and clears it.
int launch_pending_store();
// Launches the calling thread's pending write (GEMM, then store) on its own stream and
// clears it; nothing when none is pending.
int flush_pending_write();

}  // namespace starkv
