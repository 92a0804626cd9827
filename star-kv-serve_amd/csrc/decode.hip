// Paged decode over the STAR-KV low-rank cache, bf16/fp16 codes and 3.2-bit codes.
//
// Math (per request b, query head h, token l):
//   logit = scale * q . RoPE_l(U_h^T x_l)            paged_decode.py:31-102 / paged_quant.py:258-304
//         = sum_r x_l[r] * ([cos_l | sin_l] . AB[r])  AB = q folded into U (paged_quant.py:241-255,
//                                                      kv_quant.py:42-50)
//   out   = (softmax(logit) @ V_codes) @ v_up_by_q[h]  paged_decode.py:105-147, 220-226
//
// MI355X design, four launches per call (all grids are functions of host ints):
// 1. setup: the per-16-lane rank-tile table, the prefix sums of the request lengths
//    and the wave plan: whole query heads dealt to the 8 waves of a workgroup,
//    largest first to the least loaded wave, so every wave owns a balanced set of
//    rank tiles and every head lives in one wave.
// 2. fold: AB for every (request, rank tile) in fp16, written in the A-operand lane
//    order of v_mfma_f32_16x16x32_f16, so the decode kernel loads it straight into
//    its final registers.
// 3. decode: one persistent workgroup (8 waves) per CU. The requests' tokens are laid
//    end to end and cut into `grid` equal contiguous ranges, so every workgroup
//    streams the same number of cache rows whatever the lengths are; a range that
//    crosses a request boundary emits one split-K partial per request. A page is 16
//    tokens. Its 16 cos/sin rows and its rows are copied global->LDS by buffer loads
//    with the LDS bit (16 bytes per lane, no VALU address work: every lane's offset
//    inside a page is fixed for the whole kernel), three pages in flight. The only
//    workgroup barrier per page hands a page buffer over; everything else is wave
//    local. Each wave holds its heads' rank tiles of AB in VGPRs; per tile,
//    z = AB . [cos|sin]^T runs on MFMA with the page's 16 positions as N, and each lane
//    folds its 4 z values with its 4 codes. Four tiles' partial logits are summed over
//    the wave's row groups in one go with the gfx950 lane swaps. The online softmax of
//    the wave's heads runs one head per 16-lane row (lazy running max: the reference
//    point moves only when a logit exceeds it by 2^8), and P[heads, 16] @ V[16, v_rank]
//    runs on v_mfma_f32_4x4x4 (P broadcast from lanes 0-3, one V column per lane) into
//    per-wave accumulators. decode_lowrank.hip holds the bf16/fp16 kernel and
//    decode_quant.hip the 3.2-bit one, which folds the V scales into P and runs P @ V
//    one page behind over a V table expanded once per page.
// 4. merge: per (request, head) log-sum-exp of the partials, then the lift through
//    v_up_by_q.
#include <vector>

#include "decode_common.hpp"

namespace starkv {

// ---------------------------------------------------------------------------
// 1. setup: tile table, prefix sums and wave plan. One workgroup of 1024 threads.
// ---------------------------------------------------------------------------
// Wave-level integer reductions with DPP (the wave plan's steps are chains of them).
template <int CTL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTL, 0xF, 0xF, true);
}

// Min / max over lanes 0 .. 7 (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror), as a
// wave-uniform value. Every lane of the wave must be active.
__device__ __forceinline__ int lanes8_min(int v) {
    v = min(v, dpp_i<0xB1>(v));
    v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0x141>(v));
    return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ int lanes8_max(int v) {
    v = max(v, dpp_i<0xB1>(v));
    v = max(v, dpp_i<0x4E>(v));
    v = max(v, dpp_i<0x141>(v));
    return __builtin_amdgcn_readfirstlane(v);
}

// Min over all 64 lanes: within each row of 16 with DPP, then over the 4 rows.
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_i<0xB1>(v));
    v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0x141>(v));
    v = min(v, dpp_i<0x140>(v));
    const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return min(min(r0, r1), min(r2, r3));
}
__global__ __launch_bounds__(1024) void setup_kernel(const int32_t* __restrict__ seq_lens, int n, int max_seq_len,
                                                     int grid, int Hq, int Hkv, int TT,
                                                     const int32_t* __restrict__ k_ranks,
                                                     const int32_t* __restrict__ k_offsets,
                                                     const int32_t* __restrict__ t_head,
                                                     const int32_t* __restrict__ t_nout,
                                                     const int32_t* __restrict__ t_last, int qorder,
                                                     uint8_t* __restrict__ ws, size_t ws_tiles, size_t ws_plan) {
    __shared__ int s_wsum[16];
    __shared__ int s_total;
    __shared__ int s_hf[MAX_H], s_hn[MAX_H];
    __shared__ int s_rank[MAX_H], s_off[MAX_H];        // k_ranks, k_offsets (bf16/fp16)
    __shared__ int s_thead[MAX_TT], s_tmeta[MAX_TT];   // t_head, nout | last << 8 (3.2-bit)
    __shared__ int s_tword[MAX_TT];                    // per tile: code tile | outlier ranks << 13
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int* hdr = (int*)ws;
    int4* tiles = (int4*)(ws + ws_tiles);
    int* plan = (int*)(ws + ws_plan);

    // Every global input is read at once, up front: the steps below only use LDS.
    const int a = tid < n ? min(max(seq_lens[tid], 0), max_seq_len) : 0;
    if (t_head) {
        if (tid < TT) {
            s_thead[tid] = t_head[tid];
            s_tmeta[tid] = t_nout[tid] | ((t_last[tid] != 0) << 8);
        }
    } else if (tid < Hkv) {
        s_rank[tid] = k_ranks[tid];
        s_off[tid] = k_offsets[tid];
    }

    // Prefix sums of min(max(seq_len, 0), max_seq_len) over n <= 1024 requests.
    int s = a;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(s, o, 64);
        if (lane >= o) s += y;
    }
    if (lane == 63) s_wsum[wave] = s;
    __syncthreads();
    int off = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) off += w < wave ? s_wsum[w] : 0;
    if (tid < n) hdr[2 + tid] = off + s;
    if (tid == 0) hdr[1] = 0;
    if (tid == 1023) s_total = off + s;

    // Tile table and (first tile, tiles) per query head.
    if (t_head) {  // 3.2-bit: the k_tables arrays, lanes contiguous, MHA
        for (int t = tid; t < TT; t += blockDim.x) {
            tiles[t] = make_int4(s_thead[t], 16 * t, 16 | ((s_tmeta[t] & 255) << 8) | ((s_tmeta[t] >> 8) << 16),
                                 s_thead[t]);
            s_tword[t] = t | (min(s_tmeta[t] & 255, 16) << 13);
        }
        if (tid < Hq) {
            int first = -1, cnt = 0;
            for (int t = 0; t < TT; ++t)
                if (s_thead[t] == tid) { if (first < 0) first = t; ++cnt; }
            s_hf[tid] = first < 0 ? 0 : first;
            s_hn[tid] = cnt;
        }
    } else if (tid < Hq) {  // bf16/fp16: ceil(rank / 16) tiles per query head, kv = h / group
        const int grp = Hq / Hkv, kv = tid / grp;
        int t0 = 0;  // tiles of the query heads before this one: whole groups, then this group's
        for (int k = 0; k < kv; ++k) t0 += grp * ((s_rank[k] + 15) >> 4);
        const int R = s_rank[kv], o = s_off[kv];
        const int nt = (R + 15) >> 4;
        t0 += (tid - kv * grp) * nt;
        int cnt = 0;
        for (int j = 0; j < nt && t0 + j < TT; ++j, ++cnt) {
            tiles[t0 + j] = make_int4(tid, o + 16 * j, min(16, R - 16 * j) | ((j == nt - 1) << 16), kv);
            s_tword[t0 + j] = (o >> 4) + j;
        }
        s_hf[tid] = min(t0, TT);
        s_hn[tid] = cnt;
    }
    __syncthreads();
    if (tid == 0) hdr[0] = (s_total + grid - 1) / grid;

    // Wave plan. Heads sorted by decreasing tile count (ties: lower head first) are dealt
    // to the 8 waves in snake order (0..7, 7..0, 0..7, ...), so every wave takes
    // ceil(Hq / 8) or fewer heads (one head per 16-lane row of the softmax) and the big
    // heads pair with small ones; then swaps between the most loaded wave and another
    // lower the maximum while they can. Wave 0 does it in registers.
    __shared__ int s_pos[MAX_H];
    if (tid < Hq) {
        int rank = 0;
        const int mine = s_hn[tid];
#pragma unroll 8
        for (int h = 0; h < Hq; ++h) rank += s_hn[h] > mine || (s_hn[h] == mine && h < tid);
        s_pos[tid] = rank;
    }
    __syncthreads();
    if (wave == 0) {
        // Lane h < Hq: head h's tile count, first tile, order position and wave; lane
        // w < 8: wave w's tile load.
        const int hsz = lane < Hq ? s_hn[lane] : 0;
        const int hfirst = lane < Hq ? s_hf[lane] : 0;
        const int pos = lane < Hq ? s_pos[lane] : 0;
        const int round = pos / NWAVE, col = pos % NWAVE;
        int hwave = lane < Hq ? ((round & 1) ? NWAVE - 1 - col : col) : -1;
        int load = 0;
        for (int h = 0; h < Hq; ++h)  // wave loads
            load += __builtin_amdgcn_readlane(hwave, h) == lane ? __builtin_amdgcn_readlane(hsz, h) : 0;
        const int target = (TT + NWAVE - 1) / NWAVE;
        for (int it = 0; it < 64; ++it) {
            const int kmax = lanes8_max(lane < NWAVE ? (load << 8) | lane : -1);  // most loaded wave A
            const int A = kmax & 255, la = kmax >> 8;
            if (la <= target) break;
            // Candidate swaps: a head ha of A with this lane's head hb of another wave B.
            const int lb = __builtin_amdgcn_ds_bpermute(max(hwave, 0) * 4, load);  // load of hb's wave
            uint64_t inA = __builtin_amdgcn_ballot_w64(lane < Hq && hwave == A);
            int best = 0x7fffffff;
            while (inA) {
                const int ha = __builtin_ctzll(inA);
                inA &= inA - 1;
                const int d = __builtin_amdgcn_readlane(hsz, ha) - hsz;
                if (lane < Hq && hwave != A && d > 0 && lb + d < la)
                    best = min(best, (max(la - d, lb + d) << 16) | (ha << 8) | lane);
            }
            best = wave_min_i(best);
            if (best == 0x7fffffff) break;
            const int ha = (best >> 8) & 255, hb = best & 255;
            const int B = __builtin_amdgcn_readlane(hwave, hb);
            const int d = __builtin_amdgcn_readlane(hsz, ha) - __builtin_amdgcn_readlane(hsz, hb);
            if (lane == ha) hwave = B;
            if (lane == hb) hwave = A;
            if (lane == A) load -= d;
            if (lane == B) load += d;
        }
        const int ok = lanes8_max(lane < NWAVE ? load : 0) <= MAX_SLOTS;
        // Each head's place in its wave's plan: k = its wave's heads before it in the size
        // order, sl = their tiles, nfb = those of them with tiles, nnb = their tiles past
        // their first; over its whole wave: nfh heads with tiles, the largest head mxh.
        // Lane w < 8 also counts its wave's heads, tiles, heads with tiles, largest head.
        int k = 0, sl = 0, nfb = 0, nnb = 0, nfh = 0, mxh = 0, nhw = 0, ntw = 0, nfw = 0, mxw = 0;
        for (int h = 0; h < Hq; ++h) {
            const int wh = __builtin_amdgcn_readlane(hwave, h), ph = __builtin_amdgcn_readlane(pos, h);
            const int zh = __builtin_amdgcn_readlane(hsz, h);
            if (wh == hwave && ph < pos) { ++k; sl += zh; nfb += zh > 0; nnb += max(zh - 1, 0); }
            if (wh == hwave) { nfh += zh > 0; mxh = max(mxh, zh); }
            if (wh == lane) { ++nhw; ntw += zh; nfw += zh > 0; mxw = max(mxw, zh); }
        }
        // Clear the 8 plans, then every head writes its own entries (same wave: in order).
        for (int i = lane; i < NWAVE * PLAN_STRIDE; i += 64) plan[i] = 0;
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): the clears land first
        if (lane < Hq && ok) {
            int* pw = plan + hwave * PLAN_STRIDE;
            pw[32 + k] = lane;
            pw[40 + k] = sl;
            pw[48 + k] = hsz;
            for (int j = 0; j < hsz; ++j) {
                pw[8 + sl + j] = hfirst + j;
                // The decode kernel's slot order: plan order, or for the 3.2-bit kernel the
                // heads' first tiles first (the ones with outlier ranks), then the rest.
                const int ks = qorder ? (j == 0 ? nfb : nfh + nnb + j - 1) : sl + j;
                const int row = mxh <= 4 ? 4 * k + j : sl + j;  // slot_row()'s partial-logit row
                pw[PW_SLOTS + ks] = slot_word(s_tword[hfirst + j], row, k, hfirst + j);
            }
        }
        if (lane < NWAVE) {
            int* pw = plan + lane * PLAN_STRIDE;
            pw[0] = ok ? ntw : 0;
            pw[1] = ok ? nhw : 0;
            pw[2] = ok ? nfw : 0;
            pw[3] = mxw <= 4;
            for (int s = ok ? ntw : 0; s < MAX_SLOTS; ++s)  // slots past the wave's tiles: tile 0, the spare row
                pw[PW_SLOTS + s] = slot_word(s_tword[0] & SW_CODE_MASK, MAX_SLOTS, 0, 0);
        }
        if (lane == 0) plan[NWAVE * PLAN_STRIDE] = ok;
    }
}

// ---------------------------------------------------------------------------
// 2. fold: AB[b][t][ks][lane] = 8 fp16 of tile row m = lane & 15, columns
//    32 ks + 8 (lane >> 4) .. +8, scaled by scale*log2(e); rows past the head's rank
//    are zero (paged_decode.py:79-81 masks them). Row m holds rank m of the tile, or,
//    for the 3.2-bit cache (perm = 1), rank 2 (m >> 2) + ((m >> 1) & 1) + 8 (m & 1),
//    scaled by 1/16 when m & 2: then the z values a lane receives (rows 4g .. 4g+3)
//    are ranks 2g, 2g+8, 2g+1, 2g+9, the low and high nibbles of bytes g and g+4 of
//    the tile's 8 code bytes (the high nibbles are read as 16 n).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fold_tiles_kernel(const void* __restrict__ q, int64_t q_s0, int64_t q_s1,
                                                         int q_dt, const void* __restrict__ k_up, int64_t ku_s0,
                                                         int ku_dt, const uint8_t* __restrict__ ws_tiles_p, int TT,
                                                         float sc, int perm, uint8_t* __restrict__ ab) {
    const int b = blockIdx.y;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // (tile, k2, lane)
    const int t = idx >> 7, k2 = (idx >> 6) & 1, lane = idx & 63;
    if (t >= TT) return;
    const int4 tm = ((const int4*)ws_tiles_p)[t];
    const int m = lane & 15, lg = lane >> 4;
    const int rr = perm ? 2 * (m >> 2) + ((m >> 1) & 1) + 8 * (m & 1) : m;
    const int c0 = 32 * k2 + 8 * lg;
    const int64_t ur = (int64_t)(tm.y + rr) * ku_s0;
    const int64_t qh = (int64_t)b * q_s0 + (int64_t)tm.x * q_s1;
    const float s = rr < (tm.z & 255) ? (perm && (m & 2) ? sc * 0.0625f : sc) : 0.f;
    float u0[8], u1[8], q0[8], q1[8];
    load8_f(k_up, ur + c0, ku_dt, u0);
    load8_f(k_up, ur + c0 + 64, ku_dt, u1);
    load8_f(q, qh + c0, q_dt, q0);
    load8_f(q, qh + c0 + 64, q_dt, q1);
    half8_t a, bb;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (_Float16)((q0[e] * u0[e] + q1[e] * u1[e]) * s);
        bb[e] = (_Float16)((q1[e] * u0[e] - q0[e] * u1[e]) * s);
    }
    half8_t* o = (half8_t*)(ab + ((size_t)b * TT + t) * AB_TILE_BYTES);
    o[k2 * 64 + lane] = a;
    o[(k2 + 2) * 64 + lane] = bb;
}

// ---------------------------------------------------------------------------
// 4. merge: per (request, head) the partials' log-sum-exp, then the lift through
//    v_up_by_q. A workgroup takes one head and MERGE_REQ requests, so every row of
//    v_up_by_q[h] it reads serves MERGE_REQ outputs; the lift loop is unrolled so its
//    loads are in flight together.
// ---------------------------------------------------------------------------
constexpr int MERGE_REQ = 4;
constexpr int MERGE_MAXK = 64;  // partial slots per request whose weights are kept in LDS

template <typename WT>
__device__ __forceinline__ float load_w(const WT* p, int64_t i);
template <>
__device__ __forceinline__ float load_w<uint16_t>(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
template <>
__device__ __forceinline__ float load_w<_Float16>(const _Float16* p, int64_t i) { return (float)p[i]; }
template <>
__device__ __forceinline__ float load_w<float>(const float* p, int64_t i) { return p[i]; }

template <typename WT>
__global__ __launch_bounds__(128) void merge_kernel(const uint8_t* __restrict__ ws, size_t ws_plan, size_t ws_m,
                                                    size_t ws_l, size_t ws_acc, int n, int Hq, int v_rank,
                                                    const WT* __restrict__ vup, int64_t vu_s0, int64_t vu_s1,
                                                    void* __restrict__ out, int64_t o_s0, int64_t o_s1, int out_dt) {
    extern __shared__ float s_o[];                // [MERGE_REQ][v_rank]: merged low-rank outputs
    __shared__ float s_w[MERGE_REQ][MERGE_MAXK];  // per request: weight of each of its partials
    __shared__ float s_ml[MERGE_REQ][2];          // per request: reference max, 1 / sum
    __shared__ int s_k[MERGE_REQ][2];             // per request: first partial slot, count (0: no tokens)
    const int h = blockIdx.y, b0 = blockIdx.x * MERGE_REQ, tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int* hdr = (const int*)ws;
    const int S = hdr[0];
    const bool planned = ((const int*)(ws + ws_plan))[NWAVE * PLAN_STRIDE] != 0;
    const float* wm = (const float*)(ws + ws_m);
    const float* wl = (const float*)(ws + ws_l);
    const float* wa = (const float*)(ws + ws_acc);

    // 1. Per request (wave wv takes requests wv, wv + 2): the partials' log-sum-exp, with
    //    the lanes over the partial slots.
    for (int r = wv; r < MERGE_REQ; r += 2) {
        const int b = b0 + r;
        const int pb = b < n ? hdr[1 + b] : 0, pe = b < n ? hdr[2 + b] : 0;
        // No tokens: softmax over an empty row (NaN, as the reference). No wave plan (a
        // head assignment that does not fit): NaN as well, never a silent wrong result.
        const bool live = b < n && pe > pb && S > 0 && planned;
        const int k_lo = live ? pb / S : 0, nk = live ? (pe - 1) / S - k_lo + 1 : 0;
        float M = -INFINITY;
        for (int k = lane; k < nk; k += 64) M = fmaxf(M, wm[(int64_t)(k_lo + k + b) * Hq + h]);
        M = wave_max(M);
        float l = 0.f;
        for (int k = lane; k < nk; k += 64) {
            const int64_t sl = (int64_t)(k_lo + k + b) * Hq + h;
            l += wl[sl] * exp2f(wm[sl] - M);
        }
        l = wave_sum(l);
        for (int k = lane; k < nk && k < MERGE_MAXK; k += 64)
            s_w[r][k] = exp2f(wm[(int64_t)(k_lo + k + b) * Hq + h] - M);
        if (lane == 0) {
            s_ml[r][0] = M;
            s_ml[r][1] = 1.f / l;
            s_k[r][0] = k_lo;
            s_k[r][1] = nk;
        }
    }
    __syncthreads();

    // 2. The merged low-rank outputs: threads over (request, column).
    for (int i = tid; i < MERGE_REQ * v_rank; i += blockDim.x) {
        const int r = i / v_rank, c = i - r * v_rank, b = b0 + r;
        const int k_lo = s_k[r][0], nk = s_k[r][1];
        float a = 0.f;
#pragma unroll 4
        for (int k = 0; k < nk; ++k) {
            const int64_t sl = (int64_t)(k_lo + k + b) * Hq + h;
            const float w = k < MERGE_MAXK ? s_w[r][k] : exp2f(wm[sl] - s_ml[r][0]);
            a = fmaf(wa[sl * v_rank + c], w, a);
        }
        s_o[i] = a * s_ml[r][1];
    }
    __syncthreads();

    // 3. The lift through v_up_by_q[h]: each row serves MERGE_REQ requests.
    for (int d = tid; d < 128; d += blockDim.x) {
        float o[MERGE_REQ];
#pragma unroll
        for (int r = 0; r < MERGE_REQ; ++r) o[r] = 0.f;
        const WT* vp = vup + (int64_t)h * vu_s0 + d;
#pragma unroll 8
        for (int c = 0; c < v_rank; ++c) {
            const float v = load_w<WT>(vp, (int64_t)c * vu_s1);
#pragma unroll
            for (int r = 0; r < MERGE_REQ; ++r) o[r] = fmaf(s_o[r * v_rank + c], v, o[r]);
        }
#pragma unroll
        for (int r = 0; r < MERGE_REQ; ++r)
            if (b0 + r < n)
                store_f(out, (int64_t)(b0 + r) * o_s0 + (int64_t)h * o_s1 + d, out_dt,
                        s_k[r][1] > 0 ? o[r] : __builtin_nanf(""));
    }
}

// ---------------------------------------------------------------------------
// The reference API's standalone fold_q: AB fp16 [n, W, 128], row-major.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fold_q_kernel(const void* __restrict__ q, int64_t q_s0, int64_t q_s1,
                                                     int q_dt, const void* __restrict__ k_up, int64_t ku_s0,
                                                     int ku_dt, const int32_t* __restrict__ hol, int W, float scale,
                                                     _Float16* __restrict__ ab) {
    const int b = blockIdx.y;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // (lane r, i < 64)
    const int r = idx >> 6, i = idx & 63;
    if (r >= W) return;
    const int h = hol[r];
    const int64_t qo = (int64_t)b * q_s0 + (int64_t)h * q_s1;
    const float a0 = load_f(q, qo + i, q_dt), a1 = load_f(q, qo + i + 64, q_dt);
    const float u0 = load_f(k_up, (int64_t)r * ku_s0 + i, ku_dt), u1 = load_f(k_up, (int64_t)r * ku_s0 + i + 64, ku_dt);
    _Float16* o = ab + ((int64_t)b * W + r) * 128;
    o[i] = (_Float16)((a0 * u0 + a1 * u1) * scale);
    o[i + 64] = (_Float16)((a1 * u0 - a0 * u1) * scale);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

static int grid_for(int n, int max_seq_len) {
    const int64_t tokens = (int64_t)n * (int64_t)(max_seq_len > 0 ? max_seq_len : 1);
    int64_t want = (tokens + 255) / 256;  // at least ~16 pages per workgroup
    const int cus = device_cus();
    if (want > cus) want = cus;
    return want < 1 ? 1 : (int)want;
}

// Optional timing of the decode kernel alone (benchmarks): when armed, each call records
// a HIP event pair around the decode launch on the caller's stream.
struct DecodeProfile {
    bool on = false;
    int used = 0;
    std::vector<hipEvent_t> ev;
};
static DecodeProfile g_prof;

// log2(block_size / 16), or -1 if block_size is not 16 times a power of two.
static int block_shift(int block_size) {
    for (int s = 0; s < 16; ++s)
        if (block_size == (TILE_TOK << s)) return s;
    return -1;
}

struct CommonArgs {
    const void* q; int64_t q_s0, q_s1; int q_dt;
    const int32_t* bt; int64_t bt_s0, bt_s1;
    const int32_t* seq_lens;
    int n, Hq, Hkv, max_seq_len;
    const void* k_up; int64_t ku_s0; int w_dt;
    const int32_t* k_ranks; const int32_t* k_offsets;
    const int32_t* t_head; const int32_t* t_nout; const int32_t* t_last;
    const void* vup; int64_t vu_s0, vu_s1; int v_rank;
    const void* cs; int64_t cs_s0; int cs_dt;
    float scale;
    void* out; int64_t o_s0, o_s1; int out_dt;
    void* ws; size_t ws_bytes;
    int grid;
};

static int decode_common(DecodeParams& p, const CommonArgs& a, int fmt, int row_bytes, int TT, hipStream_t stream) {
    SKV_CHECK(a.n >= 1 && a.n <= MAX_REQ_PER_CALL, "decode: n=%d requests (1..%d per call)", a.n, MAX_REQ_PER_CALL);
    SKV_CHECK(a.Hq >= 1 && a.Hq <= MAX_H, "decode: num_heads=%d (1..%d)", a.Hq, MAX_H);
    SKV_CHECK(a.max_seq_len >= 1, "decode: max_seq_len must be >= 1");
    SKV_CHECK(a.v_rank >= 1, "decode: v_rank must be >= 1");
    SKV_CHECK(a.grid >= 1, "decode: grid must be >= 1");
    SKV_CHECK(TT >= 1 && TT <= MAX_TT, "decode: %d rank tiles (1..%d: k_width x heads per kv head <= %d)", TT,
              MAX_TT, MAX_TT * 16);
    const WsLayout wl = ws_layout(a.n, a.Hq, TT, a.v_rank, a.grid);
    SKV_CHECK(a.ws_bytes >= wl.total, "decode: workspace %zu bytes < %zu needed", a.ws_bytes, wl.total);
    SKV_CHECK(((uintptr_t)a.ws % 256) == 0, "decode: workspace must be 256-byte aligned");
    SKV_CHECK(p.bs_shift >= 0, "decode: block_size must be 16 times a power of two");
    SKV_CHECK(a.bt_s0 >= 0 && a.bt_s1 >= 0 &&
                  (int64_t)a.n * a.bt_s0 + (int64_t)(a.max_seq_len + TILE_TOK - 1) / TILE_TOK * a.bt_s1 <
                      ((int64_t)1 << 31),
              "decode: block_table strides must keep element indices below 2^31");
    SKV_CHECK(((uintptr_t)p.cache % 16) == 0 && p.c_s0 % 16 == 0 && p.c_s1 % 16 == 0,
              "decode: cache base and byte strides must be 16-byte aligned (c_s0=%lld c_s1=%lld)", (long long)p.c_s0,
              (long long)p.c_s1);
    SKV_CHECK(row_bytes % 16 == 0, "decode: cache row (%d bytes) must be a multiple of 16 bytes", row_bytes);
    SKV_CHECK(p.c_s1 >= row_bytes, "decode: slot stride %lld < row bytes %d", (long long)p.c_s1, row_bytes);
    SKV_CHECK(p.c_s1 * TILE_TOK < ((int64_t)1 << 31), "decode: 16 slots span %lld bytes (>= 2^31)",
              (long long)(p.c_s1 * TILE_TOK));
    SKV_CHECK(a.cs_dt == STARKV_F16, "decode: cos_sin must be fp16 (convert the table once; it is exact for bf16)");
    SKV_CHECK(a.cs_s0 % 8 == 0 && a.cs_s0 >= 128 && a.cs_s0 * 2 * TILE_TOK < ((int64_t)1 << 31) &&
                  ((uintptr_t)a.cs % 16) == 0,
              "decode: cos_sin rows must be 16-byte aligned with stride >= 128");
    SKV_CHECK(a.q_s1 % 8 == 0 && a.q_s0 % 8 == 0 && ((uintptr_t)a.q % 16) == 0,
              "decode: query rows must be 16-byte aligned (strides multiples of 8)");
    SKV_CHECK(a.ku_s0 % 8 == 0 && ((uintptr_t)a.k_up % 16) == 0, "decode: k_up rows must be 16-byte aligned");
    const int nb = (a.v_rank + 63) / 64;
    SKV_CHECK(nb <= 4, "decode: v_rank %d > 256", a.v_rank);

    p.bt = a.bt; p.bt_s0 = (int)a.bt_s0; p.bt_s1 = (int)a.bt_s1;
    p.n = a.n; p.Hq = a.Hq; p.TT = TT; p.v_rank = a.v_rank;
    p.cs = (const uint8_t*)a.cs; p.cs_s0b = (int)(a.cs_s0 * 2);
    p.row_g = row_bytes / 16;
    int qnb = 0;
    if (fmt == FMT_Q4) {
        qnb = quant_v_blocks(a.v_rank, p.v_nout);
        SKV_CHECK(qnb > 0, "decode: v_rank %d needs more than 5 P @ V blocks", a.v_rank);
        SKV_CHECK(quant_copies(row_bytes) > 0 && quant_lds_bytes(row_bytes, qnb) <= quant_lds_limit(),
                  "decode: a 3.2-bit page of %d-byte rows (v_rank %d) does not fit in LDS", row_bytes, a.v_rank);
        p.nch = quant_chunks(row_bytes);
        p.lds_bytes = quant_lds_bytes(row_bytes, qnb);
    } else {
        SKV_CHECK(lowrank_copies(p.k_width, nb) > 0,
                  "decode: a page of k_width %d and v_rank %d needs more than 64 KB of LDS", p.k_width,
                  a.v_rank);
        p.nch = lowrank_chunks(p.k_width, nb);
        p.lds_bytes = lowrank_lds_bytes(p.k_width, nb);
    }
    p.ws = (uint8_t*)a.ws;
    p.ws_tiles = wl.tiles; p.ws_plan = wl.plan; p.ws_ab = wl.ab;
    p.ws_m = wl.m; p.ws_l = wl.l; p.ws_acc = wl.acc;

    hipLaunchKernelGGL(setup_kernel, dim3(1), dim3(1024), 0, stream, a.seq_lens, a.n, a.max_seq_len, a.grid, a.Hq,
                       a.Hkv, TT, a.k_ranks, a.k_offsets, a.t_head, a.t_nout, a.t_last, fmt == FMT_Q4 ? 1 : 0, p.ws,
                       wl.tiles, wl.plan);
    SKV_HIP(hipGetLastError());
    hipLaunchKernelGGL(fold_tiles_kernel, dim3((TT * 128 + 255) / 256, a.n), dim3(256), 0, stream, a.q, a.q_s0,
                       a.q_s1, a.q_dt, a.k_up, a.ku_s0, a.w_dt, (const uint8_t*)p.ws + wl.tiles, TT,
                       a.scale * LOG2E, fmt == FMT_Q4 ? 1 : 0, p.ws + wl.ab);
    SKV_HIP(hipGetLastError());
    const bool timed = g_prof.on && 2 * g_prof.used + 1 < (int)g_prof.ev.size();
    if (timed) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used], stream));
    int rc = fmt == FMT_Q4 ? launch_quant(p, qnb, a.grid, stream) : launch_lowrank(p, fmt, nb, a.grid, stream);
    if (rc) return rc;
    SKV_HIP(hipGetLastError());
    if (timed) {
        SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used + 1], stream));
        ++g_prof.used;
    }
    const dim3 mgrid((a.n + MERGE_REQ - 1) / MERGE_REQ, a.Hq);
    const size_t mlds = (size_t)MERGE_REQ * a.v_rank * 4;
    if (a.w_dt == STARKV_BF16)
        hipLaunchKernelGGL(merge_kernel<uint16_t>, mgrid, dim3(128), mlds, stream, (const uint8_t*)p.ws, wl.plan, wl.m,
                           wl.l, wl.acc, a.n, a.Hq, a.v_rank, (const uint16_t*)a.vup, a.vu_s0, a.vu_s1, a.out, a.o_s0,
                           a.o_s1, a.out_dt);
    else if (a.w_dt == STARKV_F16)
        hipLaunchKernelGGL(merge_kernel<_Float16>, mgrid, dim3(128), mlds, stream, (const uint8_t*)p.ws, wl.plan, wl.m,
                           wl.l, wl.acc, a.n, a.Hq, a.v_rank, (const _Float16*)a.vup, a.vu_s0, a.vu_s1, a.out, a.o_s0,
                           a.o_s1, a.out_dt);
    else
        hipLaunchKernelGGL(merge_kernel<float>, mgrid, dim3(128), mlds, stream, (const uint8_t*)p.ws, wl.plan, wl.m,
                           wl.l, wl.acc, a.n, a.Hq, a.v_rank, (const float*)a.vup, a.vu_s0, a.vu_s1, a.out, a.o_s0,
                           a.o_s1, a.out_dt);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

}  // namespace starkv

using namespace starkv;

extern "C" {

int starkv_decode_grid(int n, int max_seq_len) { return grid_for(n, max_seq_len); }

int starkv_profile_begin(int max_calls) {
    clear_error();
    SKV_CHECK(max_calls >= 1 && max_calls <= 100000, "profile_begin: max_calls %d", max_calls);
    for (hipEvent_t e : g_prof.ev) (void)hipEventDestroy(e);
    g_prof.ev.assign(2 * (size_t)max_calls, nullptr);
    for (auto& e : g_prof.ev) SKV_HIP(hipEventCreate(&e));
    g_prof.used = 0;
    g_prof.on = true;
    return STARKV_OK;
}

int starkv_profile_end(double* decode_ms_sum, int* calls) {
    clear_error();
    g_prof.on = false;
    double sum = 0.0;
    for (int i = 0; i < g_prof.used; ++i) {
        SKV_HIP(hipEventSynchronize(g_prof.ev[2 * i + 1]));
        float ms = 0.f;
        SKV_HIP(hipEventElapsedTime(&ms, g_prof.ev[2 * i], g_prof.ev[2 * i + 1]));
        sum += ms;
    }
    if (decode_ms_sum) *decode_ms_sum = sum;
    if (calls) *calls = g_prof.used;
    g_prof.used = 0;
    return STARKV_OK;
}

size_t starkv_decode_workspace_bytes(int n, int num_heads, int k_tiles, int v_rank, int grid) {
    return ws_layout(n, num_heads, k_tiles, v_rank, grid).total;
}

int starkv_fold_q(void* stream, const void* q, int64_t q_s0, int64_t q_s1, int q_dtype, const void* k_up,
                  int64_t ku_s0, int ku_dtype, const int32_t* head_of_lane, int n, int k_width, float scale,
                  void* ab) {
    clear_error();
    SKV_CHECK(n >= 0 && k_width >= 0, "fold_q: negative size");
    if (n == 0 || k_width == 0) return STARKV_OK;
    SKV_CHECK(q && k_up && head_of_lane && ab, "fold_q: null pointer");
    dim3 grid((k_width * 64 + 255) / 256, n);
    hipLaunchKernelGGL(fold_q_kernel, grid, dim3(256), 0, (hipStream_t)stream, q, q_s0, q_s1, q_dtype, k_up, ku_s0,
                       ku_dtype, head_of_lane, k_width, scale, (_Float16*)ab);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

int starkv_lowrank_decode(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                          const void* kv_cache, int64_t c_s0, int64_t c_s1, int code_dtype, int block_size,
                          const int32_t* block_table, int64_t bt_s0, int64_t bt_s1, const int32_t* seq_lens, int n,
                          int num_heads, int num_kv_heads, int max_seq_len, const void* k_up, int64_t ku_s0,
                          int w_dtype, const int32_t* k_ranks, const int32_t* k_head_offsets, int k_width,
                          const void* v_up_by_q, int64_t vu_s0, int64_t vu_s1, int v_rank, const void* cos_sin,
                          int64_t cs_s0, int cs_dtype, float scale, void* out, int64_t o_s0, int64_t o_s1,
                          int out_dtype, void* workspace, size_t workspace_bytes, int grid) {
    clear_error();
    SKV_CHECK(code_dtype == STARKV_BF16 || code_dtype == STARKV_F16, "lowrank_decode: codes must be bf16 or fp16");
    SKV_CHECK(num_kv_heads >= 1 && num_heads % num_kv_heads == 0, "lowrank_decode: num_heads %% num_kv_heads != 0");
    SKV_CHECK(k_width >= 16 && k_width % 16 == 0, "lowrank_decode: k_width %d must be a positive multiple of 16",
              k_width);
    SKV_CHECK(query && kv_cache && block_table && seq_lens && k_up && k_ranks && k_head_offsets && v_up_by_q &&
                  cos_sin && out && workspace,
              "lowrank_decode: null pointer");
    DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.cache = (const uint8_t*)kv_cache;
    p.c_s0 = c_s0 * 2;
    p.c_s1 = c_s1 * 2;
    p.bs_shift = block_shift(block_size);
    p.k_width = k_width;
    CommonArgs a{query, q_s0, q_s1, q_dtype, block_table, bt_s0, bt_s1, seq_lens, n, num_heads, num_kv_heads,
                 max_seq_len, k_up, ku_s0, w_dtype, k_ranks, k_head_offsets, nullptr, nullptr, nullptr,
                 v_up_by_q, vu_s0, vu_s1, v_rank, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1, out_dtype,
                 workspace, workspace_bytes, grid};
    const int TT = (num_heads / num_kv_heads) * (k_width / 16);
    return decode_common(p, a, code_dtype == STARKV_BF16 ? FMT_BF16 : FMT_F16, (k_width + v_rank) * 2, TT,
                         (hipStream_t)stream);
}

int starkv_quant_decode(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                        const uint8_t* kv_cache, int64_t c_s0, int64_t c_s1, int block_size,
                        const int32_t* block_table, int64_t bt_s0, int64_t bt_s1, const int32_t* seq_lens, int n,
                        int num_heads, int max_seq_len, int k_width, int v_rank, int row_bytes, const void* k_up,
                        int64_t ku_s0, int w_dtype, const int32_t* tile_head, const int32_t* tile_nout,
                        const int32_t* tile_last, const void* v_up_by_q, int64_t vu_s0, int64_t vu_s1,
                        const void* cos_sin, int64_t cs_s0, int cs_dtype, float scale, void* out, int64_t o_s0,
                        int64_t o_s1, int out_dtype, void* workspace, size_t workspace_bytes, int grid) {
    clear_error();
    SKV_CHECK(k_width >= 16 && k_width % 16 == 0, "quant_decode: k_width %d must be a positive multiple of 16",
              k_width);
    SKV_CHECK(query && kv_cache && block_table && seq_lens && k_up && tile_head && tile_nout && tile_last &&
                  v_up_by_q && cos_sin && out && workspace,
              "quant_decode: null pointer");
    DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.cache = kv_cache;
    p.c_s0 = c_s0;
    p.c_s1 = c_s1;
    p.bs_shift = block_shift(block_size);
    p.k_width = k_width;
    const int v_nout = (int)(0.2 * (double)v_rank);
    p.v_nout = v_nout;
    p.v_nbo = (v_nout + 1) / 2;
    p.ks_off = k_width / 2;
    p.vs_off = p.ks_off + 4 * num_heads;
    p.vq_off = p.vs_off + 4;
    const int v_bytes = p.v_nbo + (v_rank - v_nout + 1) / 2;
    const int nbytes = (p.vq_off + v_bytes + 15) / 16 * 16;
    SKV_CHECK(row_bytes == nbytes, "quant_decode: row_bytes %d != QuantRow.nbytes %d", row_bytes, nbytes);
    CommonArgs a{query, q_s0, q_s1, q_dtype, block_table, bt_s0, bt_s1, seq_lens, n, num_heads, num_heads,
                 max_seq_len, k_up, ku_s0, w_dtype, nullptr, nullptr, tile_head, tile_nout, tile_last,
                 v_up_by_q, vu_s0, vu_s1, v_rank, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1, out_dtype,
                 workspace, workspace_bytes, grid};
    return decode_common(p, a, FMT_Q4, row_bytes, k_width / 16, (hipStream_t)stream);
}

}  // extern "C"
