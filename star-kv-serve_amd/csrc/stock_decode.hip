// Uncompressed paged decode attention: the stock bf16/fp16 comparator, and the
// attention of the layers a STAR-KV checkpoint leaves uncompressed (the reference runs
// those on vLLM's own backend: starkv_serve/model.py:77-81 builds LlamaAttention for
// them). Decode only: one query token per request attends to its first seq_len cached
// tokens.
//
// Cache layout (vLLM's per-layer key / value caches): [num_blocks, block_size, H_kv, 128]
// bf16 or fp16, element strides (c_s0, c_s1, c_s2), last dimension contiguous.
//
// stock_decode_kernel: one workgroup of 4 waves per (request, group of G query heads of
// one KV head (G = 1 or 2), split of the request's pages). A page is 16 tokens of one
// block. Lane l of a wave takes token
// l / 4 of a page and head dimensions 32 (l % 4) .. + 31: it loads 64 bytes of K and 64
// of V per page (both pages of a pair loaded before either is used), forms its part of
// q . k for each of the workgroup's G query heads, sums it over its 4 lanes, and keeps an
// online softmax (log2 domain) and 32 accumulators per query head. Waves take pages
// w, w + 4, ...; at the end the 16 token lanes of each dimension chunk are summed, the
// 4 waves merged by log-sum-exp in LDS, and the result is written (one split) or stored
// as a partial (m, l, acc[128]) that stock_merge_kernel combines.
#include <algorithm>

#include "common.hpp"

namespace starkv {

namespace {

constexpr int ST_THR = 256;
constexpr float ST_LOG2E = 1.4426950408889634f;

struct StockParams {
    const void* q; int64_t q_s0, q_s1; int q_dt;
    const uint16_t* kc; const uint16_t* vc; int64_t c_s0, c_s1, c_s2;  // elements
    int bs_shift;
    const int32_t* bt; int64_t bt_s0, bt_s1;
    const int32_t* seq_lens;
    int n, Hq, Hkv, max_seq_len, splits, pps;  // pps: pages per split
    float sc;                                  // scale * log2(e)
    float* part;                               // [n][Hq][splits][2 + 128]
    void* out; int64_t o_s0, o_s1; int out_dt;
};

template <int CDT>
__device__ __forceinline__ void cvt8(const uint4& w, float* o) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (CDT == STARKV_BF16) {
            o[2 * k] = __uint_as_float(ws[k] << 16);
            o[2 * k + 1] = __uint_as_float(ws[k] & 0xffff0000u);
        } else {
            const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(ws[k] & 0xffffu));
            const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(ws[k] >> 16));
            o[2 * k] = (float)lo;
            o[2 * k + 1] = (float)hi;
        }
    }
}

// 32 head dimensions (64 bytes) of one token row, or zeros for a token past the end.
__device__ __forceinline__ void load_row(const uint16_t* p, bool ok, uint4 (&r)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = ok ? ((const uint4*)p)[i] : make_uint4(0, 0, 0, 0);
}

template <int CDT, int G>
__global__ __launch_bounds__(ST_THR) void stock_decode_kernel(const StockParams p) {
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_acc[4][G][128];
    const int s = blockIdx.x, b = blockIdx.z;
    const int hq0 = blockIdx.y * G;                 // the workgroup's first query head
    const int h = hq0 / (p.Hq / p.Hkv);             // its KV head
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = lane >> 2, c = lane & 3;
    const int L = min(max(p.seq_lens[b], 0), p.max_seq_len);
    const int pages = (L + 15) >> 4;
    const int k0 = s * p.pps, k1 = min(k0 + p.pps, pages);

    float qv[G][32];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t qo = (int64_t)b * p.q_s0 + (int64_t)(hq0 + g) * p.q_s1 + 32 * c;
#pragma unroll
        for (int i = 0; i < 32; i += 8) {
            float f[8];
            load8_f(p.q, qo + i, p.q_dt, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[g][i + e] = f[e] * p.sc;
        }
    }
    float m[G], l[G], acc[G][32];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) acc[g][i] = 0.f;
    }
    const int mask = (1 << p.bs_shift) - 1;
    const uint16_t* kh = p.kc + (int64_t)h * p.c_s2 + 32 * c;
    const uint16_t* vh = p.vc + (int64_t)h * p.c_s2 + 32 * c;
    auto row_off = [&](int k) {
        const int blk = p.bt[(int64_t)b * p.bt_s0 + (int64_t)(k >> p.bs_shift) * p.bt_s1];
        return (int64_t)blk * p.c_s0 + (int64_t)(((k & mask) << 4) + t) * p.c_s1;
    };
    auto page = [&](int k, const uint4 (&kr)[4], const uint4 (&vr)[4]) {
        const bool ok = 16 * k + t < L;
        float kf[32], vf[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            cvt8<CDT>(kr[i], kf + 8 * i);
            cvt8<CDT>(vr[i], vf + 8 * i);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            // q . k over this lane's 32 dimensions (four chains), then over the 4 lanes of
            // the token (quad permutes), then the page max over the 16 tokens: lanes of the
            // same dimension chunk are l, l + 4, l + 8, l + 12 of each row (row rotations),
            // then the 4 rows (lane swaps).
            float dd[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 32; ++i) dd[i & 3] = fmaf(qv[g][i], kf[i], dd[i & 3]);
            float d = (dd[0] + dd[1]) + (dd[2] + dd[3]);
            d += dpp_f<0xB1>(d);  // quad_perm [1,0,3,2]
            d += dpp_f<0x4E>(d);  // quad_perm [2,3,0,1]
            const float sv = ok ? d : -INFINITY;
            float mx = fmaxf(sv, dpp_f<0x128>(sv));  // row_ror:8
            mx = fmaxf(mx, dpp_f<0x124>(mx));        // row_ror:4
            mx = max_rows(mx);
            const float mn = fmaxf(m[g], mx);
            const float alpha = mn == -INFINITY ? 1.f : exp2f(m[g] - mn);
            const float pe = ok ? exp2f(sv - mn) : 0.f;
            m[g] = mn;
            l[g] = fmaf(l[g], alpha, pe);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[g][i] = fmaf(acc[g][i], alpha, pe * vf[i]);
        }
    };
    // Pages k0 + wave, k0 + wave + 4, ..., two at a time with all four rows' loads issued first.
    int k = k0 + wave;
    for (; k + 4 < k1; k += 8) {
        uint4 ka[4], va[4], kb[4], vb[4];
        const int64_t oa = row_off(k), ob = row_off(k + 4);
        load_row(kh + oa, 16 * k + t < L, ka);
        load_row(vh + oa, 16 * k + t < L, va);
        load_row(kh + ob, 16 * (k + 4) + t < L, kb);
        load_row(vh + ob, 16 * (k + 4) + t < L, vb);
        page(k, ka, va);
        page(k + 4, kb, vb);
    }
    if (k < k1) {
        uint4 ka[4], va[4];
        const int64_t oa = row_off(k);
        load_row(kh + oa, 16 * k + t < L, ka);
        load_row(vh + oa, 16 * k + t < L, va);
        page(k, ka, va);
    }
    // Sum the 16 token lanes of each dimension chunk, then merge the 4 waves.
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float lt = l[g];
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) lt += __shfl_xor(lt, o, 64);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            float v = acc[g][i];
#pragma unroll
            for (int o = 4; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
            if (lane < 4) s_acc[wave][g][32 * c + i] = v;
        }
        if (lane == 0) {
            s_m[wave][g] = m[g];
            s_l[wave][g] = lt;  // the sum over the 16 token lanes of one dimension chunk
        }
    }
    __syncthreads();
    for (int i = tid; i < G * 128; i += ST_THR) {
        const int g = i >> 7, d = i & 127;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][g]);
        float lt = 0.f, a = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float e = s_m[w][g] == -INFINITY ? 0.f : exp2f(s_m[w][g] - M);
            lt = fmaf(s_l[w][g], e, lt);
            a = fmaf(s_acc[w][g][d], e, a);
        }
        const int hq = hq0 + g;
        if (p.splits == 1) {
            store_f(p.out, (int64_t)b * p.o_s0 + (int64_t)hq * p.o_s1 + d, p.out_dt, a / lt);  // L = 0: NaN
        } else {
            float* pp = p.part + (((int64_t)b * p.Hq + hq) * p.splits + s) * 130;
            if (d == 0) {
                pp[0] = M;
                pp[1] = lt;
            }
            pp[2 + d] = a;
        }
    }
}

// One workgroup per (query head, request): the splits' maxima and sums first (thread s
// reads split s), then every dimension's weighted sum, eight splits' loads in flight.
constexpr int ST_MAX_SPLITS = 128;
__global__ __launch_bounds__(128) void stock_merge_kernel(const StockParams p) {
    __shared__ float s_e[ST_MAX_SPLITS];
    __shared__ float s_red[2][2];  // per wave: max, then weighted sum
    const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x, w = d >> 6;
    const float* pp = p.part + ((int64_t)b * p.Hq + hq) * p.splits * 130;
    const float ms = d < p.splits ? pp[d * 130] : -INFINITY;
    const float ls = d < p.splits ? pp[d * 130 + 1] : 0.f;
    const float mw = wave_max(ms);
    if ((d & 63) == 0) s_red[w][0] = mw;
    __syncthreads();
    const float M = fmaxf(s_red[0][0], s_red[1][0]);
    const float e = ms == -INFINITY ? 0.f : exp2f(ms - M);
    const float lw = wave_sum(ls * e);
    if ((d & 63) == 0) s_red[w][1] = lw;
    if (d < p.splits) s_e[d] = e;
    __syncthreads();
    const float lt = s_red[0][1] + s_red[1][1];
    float a = 0.f;
    int s = 0;
    for (; s + 8 <= p.splits; s += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = pp[(s + u) * 130 + 2 + d];
#pragma unroll
        for (int u = 0; u < 8; ++u) a = fmaf(v[u], s_e[s + u], a);
    }
    for (; s < p.splits; ++s) a = fmaf(pp[s * 130 + 2 + d], s_e[s], a);
    store_f(p.out, (int64_t)b * p.o_s0 + (int64_t)hq * p.o_s1 + d, p.out_dt, a / lt);
}

// The step's K and V rows into their slots (what vLLM's reshape_and_cache does for the
// uncompressed layers): one workgroup per token, both caches, 16 bytes per thread and
// pass. Slot -1 (a padding token) and slots past the cache write nothing.
struct StockWriteParams {
    const uint8_t* key; const uint8_t* value; int64_t k_s0, k_s1, v_s0, v_s1;  // bytes
    uint8_t* kc; uint8_t* vc; int64_t c_s0, c_s1, c_s2;                        // bytes
    int slot_shift; int64_t num_blocks;  // slot_shift = log2(block_size)
    const void* slots; int slot64;
    int Hkv;
};
constexpr int SW_THR = 256;

__global__ __launch_bounds__(SW_THR) void stock_write_kernel(const StockWriteParams p) {
    const int t = blockIdx.x;
    const int64_t slot = p.slot64 ? ((const int64_t*)p.slots)[t] : (int64_t)((const int32_t*)p.slots)[t];
    if (slot < 0 || (slot >> p.slot_shift) >= p.num_blocks) return;
    const int64_t row = (slot >> p.slot_shift) * p.c_s0 + (slot & ((1 << p.slot_shift) - 1)) * p.c_s1;
    const int per = p.Hkv * 16;  // 16-byte granules per token and cache (256 bytes per head)
    for (int i = threadIdx.x; i < 2 * per; i += SW_THR) {
        const bool v = i >= per;
        const int j = v ? i - per : i, h = j >> 4, g = j & 15;
        const uint8_t* src = (v ? p.value + t * p.v_s0 + h * p.v_s1 : p.key + t * p.k_s0 + h * p.k_s1) + 16 * g;
        uint8_t* dst = (v ? p.vc : p.kc) + row + h * p.c_s2 + 16 * g;
        *(uint4*)dst = *(const uint4*)src;
    }
}

// Query heads per workgroup: 1 (MHA) or 2 (wider groups take several workgroups per KV
// head, whose rows they read again from L2).
template <int CDT>
const void* stock_pick(int gw) {
    return gw == 1 ? (const void*)&stock_decode_kernel<CDT, 1> : (const void*)&stock_decode_kernel<CDT, 2>;
}

// Splits per (request, head group): enough workgroups to fill the device (2 per CU), at
// least 8 pages per split, at most ST_MAX_SPLITS. groups = workgroups per request and split.
int stock_splits(int n, int groups, int max_seq_len) {
    const int pages = (max_seq_len + 15) / 16;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0) cus = c;
    }
    const int64_t wgs = (int64_t)n * groups;
    // Two workgroups of the bf16 G = 1 kernel fit a CU at once (171 VGPRs: two waves per
    // SIMD): splits that make the grid one such round of the device, or a whole number of
    // them, avoid a part-full last round (one request of 16384 tokens: 52.3 us, against
    // 57.4 us with the grid sized for three).
    int s = (int)std::min<int64_t>((2 * (int64_t)cus + wgs - 1) / wgs, (int64_t)(pages + 7) / 8);
    s = std::min(s, ST_MAX_SPLITS);
    return s < 1 ? 1 : s;
}

}  // namespace

}  // namespace starkv

using namespace starkv;

extern "C" {

size_t starkv_stock_decode_workspace_bytes(int n, int num_heads, int num_kv_heads, int max_seq_len) {
    if (n < 1 || num_heads < 1 || num_kv_heads < 1 || max_seq_len < 1) return 0;
    const int splits = stock_splits(n, num_heads == num_kv_heads ? num_heads : num_heads / 2, max_seq_len);
    return splits == 1 ? 256 : (size_t)n * num_heads * splits * 130 * 4;
}

int starkv_stock_decode(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                        const void* k_cache, const void* v_cache, int64_t c_s0, int64_t c_s1, int64_t c_s2,
                        int cache_dtype, int block_size, const int32_t* block_table, int64_t bt_s0, int64_t bt_s1,
                        const int32_t* seq_lens, int n, int num_heads, int num_kv_heads, int max_seq_len,
                        float scale, void* out, int64_t o_s0, int64_t o_s1, int out_dtype, void* workspace,
                        size_t workspace_bytes) {
    clear_error();
    SKV_CHECK(n >= 0 && max_seq_len >= 1, "stock_decode: n=%d max_seq_len=%d", n, max_seq_len);
    if (n == 0) return STARKV_OK;
    SKV_CHECK(query && k_cache && v_cache && block_table && seq_lens && out && workspace,
              "stock_decode: null pointer");
    SKV_CHECK(num_kv_heads >= 1 && num_heads % num_kv_heads == 0, "stock_decode: num_heads %% num_kv_heads != 0");
    const int G = num_heads / num_kv_heads;
    SKV_CHECK(G == 1 || G == 2 || G == 4 || G == 8, "stock_decode: %d query heads per KV head (1, 2, 4 or 8)", G);
    SKV_CHECK(cache_dtype == STARKV_BF16 || cache_dtype == STARKV_F16, "stock_decode: cache must be bf16 or fp16");
    SKV_CHECK(q_dtype >= STARKV_F32 && q_dtype <= STARKV_BF16 && out_dtype >= STARKV_F32 && out_dtype <= STARKV_BF16,
              "stock_decode: query and output dtypes must be bf16, fp16 or fp32");
    int bs_shift = -1;
    for (int sft = 0; sft < 16; ++sft)
        if (block_size == (16 << sft)) bs_shift = sft;
    SKV_CHECK(bs_shift >= 0, "stock_decode: block_size must be 16 times a power of two");
    SKV_CHECK(((uintptr_t)k_cache % 16) == 0 && ((uintptr_t)v_cache % 16) == 0 && c_s0 % 8 == 0 && c_s1 % 8 == 0 &&
                  c_s2 % 8 == 0,
              "stock_decode: cache rows must be 16-byte aligned");
    SKV_CHECK(q_s0 % 8 == 0 && q_s1 % 8 == 0 && ((uintptr_t)query % 16) == 0,
              "stock_decode: query rows must be 16-byte aligned");
    const int gw = G == 1 ? 1 : 2;
    const int splits = stock_splits(n, num_heads / gw, max_seq_len);
    const size_t need = starkv_stock_decode_workspace_bytes(n, num_heads, num_kv_heads, max_seq_len);
    SKV_CHECK(workspace_bytes >= need, "stock_decode: workspace %zu bytes < %zu", workspace_bytes, need);
    StockParams p;
    p.q = query; p.q_s0 = q_s0; p.q_s1 = q_s1; p.q_dt = q_dtype;
    p.kc = (const uint16_t*)k_cache; p.vc = (const uint16_t*)v_cache;
    p.c_s0 = c_s0; p.c_s1 = c_s1; p.c_s2 = c_s2; p.bs_shift = bs_shift;
    p.bt = block_table; p.bt_s0 = bt_s0; p.bt_s1 = bt_s1; p.seq_lens = seq_lens;
    p.n = n; p.Hq = num_heads; p.Hkv = num_kv_heads; p.max_seq_len = max_seq_len; p.splits = splits;
    p.pps = ((max_seq_len + 15) / 16 + splits - 1) / splits;
    p.sc = scale * ST_LOG2E;
    p.part = (float*)workspace;
    p.out = out; p.o_s0 = o_s0; p.o_s1 = o_s1; p.out_dt = out_dtype;
    const void* fn = cache_dtype == STARKV_BF16 ? stock_pick<STARKV_BF16>(gw) : stock_pick<STARKV_F16>(gw);
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(splits, num_heads / gw, n), dim3(ST_THR), args, 0, (hipStream_t)stream));
    if (splits > 1) {
        hipLaunchKernelGGL(stock_merge_kernel, dim3(num_heads, n), dim3(128), 0, (hipStream_t)stream, p);
        SKV_HIP(hipGetLastError());
    }
    return STARKV_OK;
}

int starkv_stock_write(void* stream, const void* key, int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0,
                       int64_t v_s1, int dtype, void* k_cache, void* v_cache, int64_t c_s0, int64_t c_s1, int64_t c_s2,
                       int block_size, int64_t num_blocks, const void* slot_mapping, int slot_bits, int n,
                       int num_kv_heads) {
    clear_error();
    SKV_CHECK(n >= 0 && num_kv_heads >= 1, "stock_write: n=%d num_kv_heads=%d", n, num_kv_heads);
    if (n == 0) return STARKV_OK;
    SKV_CHECK(key && value && k_cache && v_cache && slot_mapping, "stock_write: null pointer");
    SKV_CHECK(dtype == STARKV_BF16 || dtype == STARKV_F16, "stock_write: K/V must be bf16 or fp16");
    SKV_CHECK(slot_bits == 32 || slot_bits == 64, "stock_write: slot_mapping must be int32 or int64");
    int bs_shift = -1;
    for (int sft = 0; sft < 16; ++sft)
        if (block_size == (16 << sft)) bs_shift = sft;
    SKV_CHECK(bs_shift >= 0, "stock_write: block_size must be 16 times a power of two");
    const uintptr_t al = (uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache | (uintptr_t)v_cache;
    SKV_CHECK(al % 16 == 0 && (k_s0 | k_s1 | v_s0 | v_s1 | c_s0 | c_s1 | c_s2) % 8 == 0,
              "stock_write: rows must be 16-byte aligned");
    StockWriteParams p;
    p.key = (const uint8_t*)key; p.value = (const uint8_t*)value;
    p.k_s0 = 2 * k_s0; p.k_s1 = 2 * k_s1; p.v_s0 = 2 * v_s0; p.v_s1 = 2 * v_s1;
    p.kc = (uint8_t*)k_cache; p.vc = (uint8_t*)v_cache; p.c_s0 = 2 * c_s0; p.c_s1 = 2 * c_s1; p.c_s2 = 2 * c_s2;
    p.slot_shift = bs_shift + 4; p.num_blocks = num_blocks;  // block_size = 16 << bs_shift
    p.slots = slot_mapping; p.slot64 = slot_bits == 64;
    p.Hkv = num_kv_heads;
    hipLaunchKernelGGL(stock_write_kernel, dim3(n), dim3(SW_THR), 0, (hipStream_t)stream, p);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

}  // extern "C"
