// Dense causal prefill attention of the STAR-KV attention layer (the reference runs it on
// vLLM's FlashAttention: attention.py:219-251 lifts K and V from the step's codes, then
// flash_attn_varlen_func(causal=True) over the prompts). Every prompt attends to itself
// only (no cached context): out[t, h] = softmax(scale q[t, h] . K[s .. t, h / G]) V[s .. t,
// h / G] for token t of the prompt starting at s.
//
// Inputs: q [T, Hq, 128] (bf16, fp16 or fp32; converted to fp16 on load), K and V
// [T, Hkv, 128] fp16 (the lifted keys and values, rounded once to fp16), cu_seqlens
// [P + 1] (the prompts' first tokens), and a block list: per workgroup row, (prompt,
// 128-row query block) (starkv_prefill_block_list writes it on the host).
//
// prefill_kernel: one workgroup of 4 waves per (query block of 128 rows, query head); wave
// w takes query rows 32 w .. 32 w + 31 of the block. Keys go by tiles of 64, K and V of a
// tile copied global->LDS by all waves (buffer loads that write LDS, bounded to the
// prompt's rows), the next tile in flight while one is used. The block list puts the
// blocks with the most keys first. Per tile and wave, on v_mfma_f32_32x32x16_f16:
//   S^T = K Q^T: M = 32 keys (two blocks per tile), N = the wave's 32 queries, K = the 128
//     head dimensions (8 steps); A = a K row's 8 dimensions (ds_read_b128 from a row whose
//     16-byte granules are XOR-swizzled by the row, so 16 rows hit distinct banks), B = Q
//     in registers for the whole kernel.
//   Each lane then holds 32 scores of one query (column n = lane % 32) and its partner lane
//     (lane ^ 32) the other 32: causal and prompt-end masking, an online softmax in the
//     log2 domain with a lazy reference max (it moves only when a score exceeds it by
//     2^8), one lane swap per tile for the max.
//   O^T += V^T P^T: M = 32 head dimensions (4 blocks), N = the queries, K = 16 keys (4
//     steps). The lane's P values of one step are already the B operand if the K index
//     8 h + e (h = lane / 32) stands for key 4 h + e (e < 4) or 8 + 4 h + e - 4; A = V^T with
//     the same key order, read with ds_read_b64_tr_b16 (4 key rows x 16 dimensions per
//     16-lane group, lane i receiving dimension i).
// At the end the two halves of each query's sum are added and O / l is written.
#include <algorithm>
#include <array>
#include <vector>

#include "decode_pages.hpp"

namespace starkv {

namespace {

constexpr int PF_WAVES = 4;
constexpr int PF_THR = PF_WAVES * 64;
constexpr int PF_QB = 32 * PF_WAVES;      // query rows per workgroup
constexpr int PF_KT = 64;                 // keys per tile
constexpr int PF_TILE = PF_KT * 256;      // bytes of K (or V) per tile: 64 rows x 128 fp16
constexpr int PF_BUF = 2 * PF_TILE;       // K then V
constexpr int PF_NBUF = 2;                // tile buffers: the next tile lands while one is used
constexpr int PF_CPW = 32 / PF_WAVES;     // 1 KB copies per wave per tile
constexpr float PF_LAZY = 8.f;            // log2 headroom of the reference max

typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct PrefillParams {
    const void* q; int64_t q_s0, q_s1; int q_dt;
    const uint8_t* k; const uint8_t* v; int64_t kv_s0, kv_s1;  // bytes
    const int32_t* cu;                                        // [P + 1]
    const int32_t* blocks;                                    // [nblocks][2]: prompt, query block
    int Hq, G;
    float sc;                                                 // scale * log2(e)
    void* out; int64_t o_s0, o_s1; int out_dt;                // elements
};

// Physical byte of (row, 16-byte granule g) in a K or V tile: granules XOR-swizzled by the row.
__device__ __forceinline__ uint32_t pf_addr(int row, int g) { return (uint32_t)(row * 256 + ((g ^ (row & 15)) << 4)); }

// 8 query dimensions times scale * log2(e), as fp16 (zeros past the prompt).
template <int QDT>
__device__ __forceinline__ half8_t pf_load_q(const PrefillParams& p, int64_t tok, int hq, int d0, bool ok) {
    half8_t r;
    if (!ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (_Float16)0.f;
        return r;
    }
    const int64_t off = tok * p.q_s0 + (int64_t)hq * p.q_s1 + d0;
    float f[8];
    if (QDT == STARKV_F16) {
        const half8_t x = *(const half8_t*)((const _Float16*)p.q + off);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float)x[e];
    } else if (QDT == STARKV_BF16) {
        const uint4 w = *(const uint4*)((const uint16_t*)p.q + off);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f[2 * k] = __uint_as_float(ws[k] << 16);
            f[2 * k + 1] = __uint_as_float(ws[k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = ((const float*)p.q)[off + e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)(f[e] * p.sc);
    return r;
}

// 4 transposed 16-bit elements (see the file comment).
__device__ __forceinline__ uint2 pf_tr(uint32_t addr) {
    typedef short s4_t __attribute__((ext_vector_type(4)));
    const s4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4_t*)(uintptr_t)addr);
    return __builtin_bit_cast(uint2, r);
}

template <int QDT, int ODT>
__global__ __launch_bounds__(PF_THR) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(const PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_kv[];  // two tiles of K then V
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    const int n = lane & 31, h = lane >> 5;
    // Wave-uniform (readfirstlane): the copy descriptors built from them live in SGPRs.
    const int pr = rfl(p.blocks[2 * blockIdx.x]), qblk = rfl(p.blocks[2 * blockIdx.x + 1]);
    const int s = rfl(p.cu[pr]), L = rfl(p.cu[pr + 1]) - s;
    const int hq = blockIdx.y, hk = hq / p.G;
    const int q0 = qblk * PF_QB;
    const int qw = q0 + 32 * wave;          // the wave's first query (prompt-relative)
    const int nq = min(32, L - qw);         // its rows (<= 0: none)
    const int qi = qw + n;                  // this lane's query
    const int kend = min(L, q0 + PF_QB);    // keys the workgroup needs: [0, kend)
    const int ntile = (kend + PF_KT - 1) / PF_KT;

    // Q as the B operand of S^T = K Q^T: query n, dimensions 16 ks + 8 h .. + 7.
    half8_t qb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qb[ks] = pf_load_q<QDT>(p, (int64_t)s + qi, hq, 16 * ks + 8 * h, qi < L);

    // Copies: a tile is 32 KB (K rows then V rows), 32 copies of 1 KB, PF_CPW per wave.
    // Copy c of wave w moves LDS bytes [1024 (PF_WAVES c + w), + 1024): K (or V, past
    // 16 KB) rows 4 ((PF_WAVES c + w) % 16) .. + 3; lane j writes physical granule j % 16
    // of row (j / 16) of them, i.e. logical granule (j % 16) ^ (row & 15).
    const uint32_t base = lds_addr(s_kv);
    uint32_t coff[PF_CPW];
#pragma unroll
    for (int c = 0; c < PF_CPW; ++c) {
        const int ch = PF_WAVES * c + wave;       // 1 KB chunk of the tile
        const int row = (ch % 16) * 4 + (lane >> 4);
        const int g = (lane & 15) ^ (row & 15);
        coff[c] = (uint32_t)(row * p.kv_s0 + 16 * g);
    }
    const int64_t head_off = (int64_t)hk * p.kv_s1;
    auto issue = [&](int t) {  // tile t's copies into buffer t % PF_NBUF
        const uint32_t buf = base + (uint32_t)((t % PF_NBUF) * PF_BUF);
        const int r0 = t * PF_KT;
        const int rows = max(0, min(PF_KT, L - r0));
        int4v_t rk = buffer_rsrc(p.k + ((int64_t)s + r0) * p.kv_s0 + head_off, (int)(rows * p.kv_s0));
        int4v_t rv = buffer_rsrc(p.v + ((int64_t)s + r0) * p.kv_s0 + head_off, (int)(rows * p.kv_s0));
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // uniform by construction; the copies take them in SGPRs
            rk[e] = rfl(rk[e]);
            rv[e] = rfl(rv[e]);
        }
#pragma unroll
        for (int c = 0; c < PF_CPW; ++c) {  // chunks PF_WAVES c + wave: K for the first 16, V after
            const uint32_t m0 = buf + (uint32_t)(PF_WAVES * c + wave) * 1024u;
            if (c < PF_CPW / 2)
                lds_copy16(rk, m0, coff[c]);
            else
                lds_copy16(rv, m0, coff[c]);
        }
    };

    // Per-lane LDS offsets (from a tile's K base). A of S^T: key row 32 mb + n, granule
    // 2 ks + h (block mb = 1 is 32 rows further: the same swizzle, + 8 KB).
    uint32_t ka[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) ka[ks] = pf_addr(n, 2 * ks + h);
    // A of O^T (from the tile's V base): 16-lane group q reads key rows 16 ks + 4 (q >> 1) +
    // i / 4 (and + 8) at dimensions 32 md + 16 (q & 1) + 4 (i % 4).
    const int qg = lane >> 4, li = lane & 15;
    // Step ks is 16 rows (4 KB) further with the same swizzle.
    uint32_t va[4][2];
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int row = 8 * half + 4 * (qg >> 1) + (li >> 2);
            const int dim = 32 * md + 16 * (qg & 1) + 4 * (li & 3);
            va[md][half] = (uint32_t)(row * 256 + (((dim >> 3) ^ (row & 15)) << 4) + 2 * (dim & 7));
        }

    f32x16_t o[4];
#pragma unroll
    for (int md = 0; md < 4; ++md) o[md] = (f32x16_t){};
    float m = -INFINITY, l = 0.f;

    // Two workgroups share a CU (64 KB of LDS each): with three tile buffers and 8 waves per
    // workgroup instead, one 16K-token prompt took 3.54 ms against 3.18 here.
    issue(0);
    for (int t = 0; t < ntile; ++t) {
        SKV_WAIT_VM_LGKM0(0);  // tile t has landed (this wave's copies)
        lds_barrier();         // every wave's copies of tile t; every wave done with tile t - 1
        if (t + 1 < ntile) issue(t + 1);  // into tile t - 1's buffer
        const int k0 = t * PF_KT;
        if (nq > 0 && k0 <= qw + nq - 1) {  // some key of the tile is visible to the wave
            const uint32_t kb = base + (uint32_t)((t % PF_NBUF) * PF_BUF), vb = kb + PF_TILE;
            f32x16_t sc[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                sc[mb] = (f32x16_t){};
#pragma unroll
                for (int ks = 0; ks < 8; ++ks)
                    sc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lds_ld<half8_t>(kb + 8192u * mb + ka[ks]), qb[ks],
                                                                   sc[mb], 0, 0, 0);
            }
            // Scores of this lane's query (already scaled through q): key k0 + 32 mb + 8 (r / 4) +
            // 4 h + r % 4. Only a tile that reaches past the wave's first query or the prompt's
            // end needs the causal / end mask.
            if (k0 + PF_KT - 1 > qw || k0 + PF_KT > L) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + 32 * mb + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (!(key <= qi && key < L)) sc[mb][r] = -INFINITY;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[mb][r]);
            {  // with the partner lane's half: x[0] holds lane l % 32's value, x[1] lane 32 + l % 32's
                const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
            }
            if (__builtin_amdgcn_ballot_w64(mx > m + PF_LAZY) != 0) {
                const float mn = fmaxf(m, mx);
                const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
                m = mn;
                l *= alpha;
#pragma unroll
                for (int md = 0; md < 4; ++md)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[md][r] *= alpha;
            }
            // P in fp16 as the B operand of each 16-key step: elements 8 (ks % 2) .. + 7 of block ks / 2.
            half8_t pb[4];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = sc[mb][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[mb][r] - m);
                    l += e;
                    pb[2 * mb + (r >> 3)][r & 7] = (_Float16)e;
                }
#pragma unroll
            for (int md = 0; md < 4; ++md)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const uint2 a0 = pf_tr(vb + 4096u * ks + va[md][0]), a1 = pf_tr(vb + 4096u * ks + va[md][1]);
                    const half8_t av = __builtin_bit_cast(half8_t, make_uint4(a0.x, a0.y, a1.x, a1.y));
                    o[md] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb[ks], o[md], 0, 0, 0);
                }
        }
    }
    // The query's sum over both halves, then O / l: dimensions 32 md + 8 (r / 4) + 4 h + r % 4.
    {
        const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
        l = __uint_as_float(x[0]) + __uint_as_float(x[1]);
    }
    if (qi < L && nq > 0) {
        const float inv = 1.f / l;
        const int64_t ob = ((int64_t)s + qi) * p.o_s0 + (int64_t)hq * p.o_s1;
#pragma unroll
        for (int md = 0; md < 4; ++md)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = 32 * md + 8 * j + 4 * h;
                const float v0 = o[md][4 * j] * inv, v1 = o[md][4 * j + 1] * inv;
                const float v2 = o[md][4 * j + 2] * inv, v3 = o[md][4 * j + 3] * inv;
                if (ODT == STARKV_F32) {
                    *(float4*)((float*)p.out + ob + d) = make_float4(v0, v1, v2, v3);
                } else if (ODT == STARKV_F16) {
                    const half2_t a = cvt_h2(v0, v1), b = cvt_h2(v2, v3);
                    *(uint2*)((_Float16*)p.out + ob + d) = make_uint2(h2_bits(a), h2_bits(b));
                } else {
                    const uint32_t a = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v0) |
                                       ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v1) << 16);
                    const uint32_t b = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v2) |
                                       ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v3) << 16);
                    *(uint2*)((uint16_t*)p.out + ob + d) = make_uint2(a, b);
                }
            }
    }
    SKV_WAIT_VM_LGKM0(0);  // no copy may land after the workgroup ends
}

template <int QDT>
const void* pf_pick(int odt) {
    if (odt == STARKV_F32) return (const void*)&prefill_kernel<QDT, STARKV_F32>;
    if (odt == STARKV_F16) return (const void*)&prefill_kernel<QDT, STARKV_F16>;
    return (const void*)&prefill_kernel<QDT, STARKV_BF16>;
}

}  // namespace

}  // namespace starkv

using namespace starkv;

extern "C" {

int starkv_prefill_block_list(const int32_t* cu_seqlens, int num_prompts, int32_t* blocks, int capacity) {
    // (keys, prompt, block) of every 128-row query block, the most keys first (ties in
    // prompt then block order): the longest causal rows start first and the short ones
    // fill the tail.
    if (!cu_seqlens || num_prompts < 0) return -1;
    std::vector<std::array<int, 3>> all;
    for (int i = 0; i < num_prompts; ++i) {
        const int L = cu_seqlens[i + 1] - cu_seqlens[i];
        if (L < 0) return -1;
        for (int b = 0; b * PF_QB < L; ++b) all.push_back({std::min(L, PF_QB * (b + 1)), i, b});
    }
    std::stable_sort(all.begin(), all.end(), [](const std::array<int, 3>& x, const std::array<int, 3>& y) {
        return x[0] > y[0];
    });
    if (blocks)
        for (int k = 0; k < (int)all.size() && k < capacity; ++k) {
            blocks[2 * k] = all[k][1];
            blocks[2 * k + 1] = all[k][2];
        }
    return (int)all.size();
}

int starkv_prefill_attention(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                             const void* key, const void* value, int64_t kv_s0, int64_t kv_s1, int kv_dtype,
                             const int32_t* cu_seqlens, const int32_t* blocks, int num_blocks, int num_heads,
                             int num_kv_heads, int head_size, float scale, void* out, int64_t o_s0, int64_t o_s1,
                             int out_dtype) {
    clear_error();
    SKV_CHECK(num_blocks >= 0, "prefill: num_blocks=%d", num_blocks);
    if (num_blocks == 0) return STARKV_OK;
    SKV_CHECK(query && key && value && cu_seqlens && blocks && out, "prefill: null pointer");
    SKV_CHECK(head_size == 128, "prefill: head_size %d (128 only)", head_size);
    SKV_CHECK(num_kv_heads >= 1 && num_heads >= 1 && num_heads % num_kv_heads == 0,
              "prefill: num_heads %% num_kv_heads != 0");
    SKV_CHECK(kv_dtype == STARKV_F16, "prefill: K and V must be fp16");
    SKV_CHECK(q_dtype >= STARKV_F32 && q_dtype <= STARKV_BF16 && out_dtype >= STARKV_F32 && out_dtype <= STARKV_BF16,
              "prefill: query and output dtypes must be bf16, fp16 or fp32");
    SKV_CHECK(((uintptr_t)key % 16) == 0 && ((uintptr_t)value % 16) == 0 && kv_s0 % 8 == 0 && kv_s1 % 8 == 0,
              "prefill: K and V rows must be 16-byte aligned");
    SKV_CHECK(kv_s0 * 2 * 64 < ((int64_t)1 << 31), "prefill: K / V row stride too large");
    const int qal = q_dtype == STARKV_F32 ? 4 : 8;
    SKV_CHECK(((uintptr_t)query % 16) == 0 && q_s0 % qal == 0 && q_s1 % qal == 0,
              "prefill: query rows must be 16-byte aligned");
    SKV_CHECK(o_s0 % 4 == 0 && o_s1 % 4 == 0 && ((uintptr_t)out % 16) == 0, "prefill: output rows must be aligned");
    PrefillParams p;
    p.q = query; p.q_s0 = q_s0; p.q_s1 = q_s1; p.q_dt = q_dtype;
    p.k = (const uint8_t*)key; p.v = (const uint8_t*)value;
    p.kv_s0 = kv_s0 * 2; p.kv_s1 = kv_s1 * 2;
    p.cu = cu_seqlens; p.blocks = blocks;
    p.Hq = num_heads; p.G = num_heads / num_kv_heads;
    p.sc = scale * 1.4426950408889634f;
    p.out = out; p.o_s0 = o_s0; p.o_s1 = o_s1; p.out_dt = out_dtype;
    const void* fn = q_dtype == STARKV_F32 ? pf_pick<STARKV_F32>(out_dtype)
                     : q_dtype == STARKV_F16 ? pf_pick<STARKV_F16>(out_dtype)
                                             : pf_pick<STARKV_BF16>(out_dtype);
    const int lds = PF_NBUF * PF_BUF;
    static const void* raised[16];
    static int nraised = 0;
    bool seen = false;
    for (int i = 0; i < nraised; ++i) seen = seen || raised[i] == fn;
    if (!seen) {
        SKV_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        if (nraised < 16) raised[nraised++] = fn;
    }
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(num_blocks, num_heads), dim3(PF_THR), args, (size_t)lds, (hipStream_t)stream));
    return STARKV_OK;
}

}  // extern "C"
