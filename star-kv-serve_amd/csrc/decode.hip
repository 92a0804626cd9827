// Paged decode over the STAR-KV low-rank cache, bf16/fp16 codes and 3.2-bit codes.
//
// Math (per request b, query head h, token l):
//   logit = scale * q . RoPE_l(U_h^T x_l)            paged_decode.py:31-102 / paged_quant.py:258-304
//         = sum_r x_l[r] * ([cos_l | sin_l] . AB[r])  AB = q folded into U (paged_quant.py:241-255,
//                                                      kv_quant.py:42-50)
//   out   = (softmax(logit) @ V_codes) @ v_up_by_q[h]  paged_decode.py:105-147, 220-226
//
// MI355X design, three launches per call (all grids are functions of host ints):
// 1. prep: workgroup 0 writes the prefix sums of the request lengths, workgroup 1 the
//    wave plan: whole query heads dealt to the 8 waves of a decode workgroup, so every
//    wave owns a balanced set of rank tiles and every head lives in one wave. The other
//    workgroups fold AB for every (request, rank tile) in fp16, written in the
//    A-operand lane order of v_mfma_f32_16x16x32_f16, so the decode kernel loads it
//    straight into its final registers.
// 2. decode: one persistent workgroup (8 waves) per CU. The requests' tokens are laid
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
// 3. merge: per (request, head) log-sum-exp of the partials, then the lift through
//    v_up_by_q.
// V ranks too wide for the decode kernel's P @ V (bf16/fp16 above 256, 3.2-bit above
// five 64-lane blocks) take the two-pass form of decode_wide.hip instead: the decode
// kernels run as a logits pass (K side and softmax statistics, logits stored in the
// workspace), a P @ V pass reads the logits and the V bytes, and a merge of its own
// lifts the result. Both forms take the same arguments and give the same outputs to
// within rounding.
#include <algorithm>
#include <vector>

#include "decode_common.hpp"
#include "kv_gemm.hpp"

namespace starkv {
// ---------------------------------------------------------------------------
// 1. prep: one launch of PREP_THR-thread workgroups. Workgroup 0 writes the prefix
//    sums of the request lengths, workgroup 1 the wave plan (the two side by side: the
//    plan is the longer chain); every other workgroup folds AB for two rank tiles and up
//    to PREP_REQ requests. The plan and the folds read the rank-tile table, which each
//    workgroup builds in LDS from the per-head ranks (bf16/fp16) or the per-tile arrays
//    (3.2-bit).
// ---------------------------------------------------------------------------
constexpr int PREP_THR = 256;
constexpr int PREP_REQ = 8;  // requests per fold workgroup

struct PrepArgs {
    const int32_t* seq_lens;
    int n, max_seq_len, grid, Hq, Hkv, TT, k_rows;
    const int32_t* k_ranks; const int32_t* k_offsets;                       // bf16/fp16
    const int32_t* t_head; const int32_t* t_nout; const int32_t* t_last;  // 3.2-bit (t_head set)
    int head0, code0;  // 3.2-bit head groups: the group's first head, code tile of its first tile
    const void* q; int64_t q_s0, q_s1; int q_dt;
    const void* k_up; int64_t ku_s0; int ku_dt;
    float sc;  // scale * log2(e)
    uint8_t* ws; size_t ws_plan, ws_ab;
    int tile_pairs;  // ceil(TT / 2): fold workgroups per group of PREP_REQ requests
    int fold_wgs;    // fold workgroups (after workgroups 0 and 1); the page-record ones follow
    // Page records (PageRec, one per page of every request) for the decode launches.
    PageRec* pages;
    const uint8_t* cache; int64_t c_s0, c_s1;  // bytes
    int bs_shift;
    const int32_t* bt; int64_t bt_s0, bt_s1;
};
constexpr int PREP_RECS = 4 * PREP_THR;  // page records per record workgroup

// Rank-tile table: per tile its query head, first k_up row, valid ranks (rows past them
// fold to zero) and code word (slot_word's code tile | outlier ranks << 13); per query
// head its first tile and tile count.
struct alignas(16) TileTable {
    int head[MAX_TT], row[MAX_TT], valid[MAX_TT], word[MAX_TT];
    int hf[MAX_H], hn[MAX_H];
    int rank[MAX_H], off[MAX_H], t0[MAX_H];  // bf16/fp16 kv heads: t0 = tiles of the kv heads before
};

// Fills `tt` (every thread of the workgroup calls it; it ends with a barrier).
//   bf16/fp16: query head h (kv head h / (Hq / Hkv)) has ceil(rank / 16) tiles; the
//     heads' tiles are laid out head after head, k_up rows from the kv head's offset.
//   3.2-bit: tile t belongs to head t_head[t] - head0 (a call over a group of heads
//     gets the tables from the group's first tile on), k_up rows 16 t .. 16 t + 15
//     (lanes contiguous), outlier ranks t_nout[t], code tile code0 + t.
__device__ void tile_table(const PrepArgs& a, TileTable& tt, int tid) {
    int h = 0, hp = -1, nout = 0;  // 3.2-bit: tile tid's head, tile tid - 1's head, outlier ranks
    if (a.t_head) {
        if (tid < a.TT) {
            h = min(max(a.t_head[tid] - a.head0, 0), a.Hq - 1);
            if (tid > 0) hp = min(max(a.t_head[tid - 1] - a.head0, 0), a.Hq - 1);
            nout = min(max(a.t_nout[tid], 0), 16);
        }
    } else if (tid < 64) {
        // Wave 0: the kv heads' ranks and offsets, and the tiles before each kv head (all
        // its query heads'), an exclusive lane scan (Hkv <= 32 lanes).
        const int R = tid < a.Hkv ? min(max(a.k_ranks[tid], 0), 16 * MAX_TT) : 0;
        if (tid < a.Hkv) {
            tt.rank[tid] = R;
            tt.off[tid] = a.k_offsets[tid];
        }
        const int v = (a.Hq / a.Hkv) * ((R + 15) >> 4);
        int incl = v;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (tid >= o) incl += y;
        }
        if (tid < a.Hkv) tt.t0[tid] = incl - v;
    }
    if (tid < MAX_TT) {
        tt.head[tid] = 0;
        tt.row[tid] = 0;
        tt.valid[tid] = 0;
        tt.word[tid] = 0;
    }
    if (tid < MAX_H) {
        tt.hf[tid] = 0;
        tt.hn[tid] = 0;
    }
    __syncthreads();
    if (a.t_head) {
        if (tid < a.TT) {
            tt.head[tid] = h;
            tt.row[tid] = 16 * tid;
            tt.valid[tid] = 16;
            tt.word[tid] = (a.code0 + tid) | (nout << 13);
            atomicAdd(&tt.hn[h], 1);
            if (hp != h) tt.hf[h] = tid;  // a head's tiles are contiguous
        }
    } else if (tid < a.Hq) {
        const int grp = a.Hq / a.Hkv, kv = tid / grp;
        int t0 = tt.t0[kv];  // tiles of the query heads before this one: whole groups, then this group's
        const int R = tt.rank[kv], o = tt.off[kv];
        const int nt = (R + 15) >> 4;
        t0 += (tid - kv * grp) * nt;
        int cnt = 0;
        for (int j = 0; j < nt && t0 + j < a.TT; ++j, ++cnt) {
            tt.head[t0 + j] = tid;
            tt.row[t0 + j] = min(max(o + 16 * j, 0), a.k_rows - 16);
            tt.valid[t0 + j] = min(16, R - 16 * j);
            tt.word[t0 + j] = (o >> 4) + j;
        }
        tt.hf[tid] = min(t0, a.TT);
        tt.hn[tid] = cnt;
    }
    __syncthreads();
}

// Wave-level integer reductions with DPP (the wave plan's steps are chains of them).
template <int CTL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTL, 0xF, 0xF, true);
}

// Inclusive scan over lanes 0 .. 31 (lanes 32 .. 63 get a scan of their own): row_shr 1, 2,
// 4, 8 within each row of 16, then row 1 adds lane 15 (row_bcast:15 into rows 1 and 3).
__device__ __forceinline__ void scan32(uint32_t& v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);
}

// Max over lanes 0 .. 7 (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror), as a
// wave-uniform value. Every lane of the wave must be active.
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

// The requests' page counts, min(max(seq_len, 0), max_seq_len) tokens in pages of 16, as
// an inclusive prefix: s_pp[b + 1] = pages of requests 0 .. b, s_pp[0] = 0; s_len[b] the
// clamped lengths. Every thread of the workgroup calls it (requests 4 tid .. 4 tid + 3);
// it ends with a barrier.
__device__ void page_prefix(const PrepArgs& a, int tid, int* s_pp, int* s_len) {
    __shared__ int s_wsum[PREP_THR / 64];
    const int lane = tid & 63, wave = tid >> 6;
    int v[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * tid + i;
        const int L = b < a.n ? min(max(a.seq_lens[b], 0), a.max_seq_len) : 0;
        if (b < a.n) s_len[b] = L;
        v[i] = (L + TILE_TOK - 1) / TILE_TOK;
        s += v[i];
    }
    int incl = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int run = incl - s;
#pragma unroll
    for (int w = 0; w < PREP_THR / 64; ++w) run += w < wave ? s_wsum[w] : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        run += v[i];
        if (4 * tid + i < a.n) s_pp[4 * tid + i + 1] = run;
    }
    if (tid == 0) s_pp[0] = 0;
    __syncthreads();
}

// Workgroup 0 of prep: hdr[0] = pages per decode workgroup (the last workgroups may have
// none), hdr[1 + b] = first page of request b in the concatenation, hdr[1 + n] = all pages.
__device__ void prep_prefix(const PrepArgs& a, int tid, int* s_pp, int* s_len) {
    page_prefix(a, tid, s_pp, s_len);
    int* hdr = (int*)a.ws;
    for (int b = tid; b <= a.n; b += PREP_THR) hdr[1 + b] = s_pp[b];
    if (tid == 0) hdr[0] = (s_pp[a.n] + a.grid - 1) / a.grid;
}

// Record workgroup w of prep: the records of pages w PREP_RECS .. (w + 1) PREP_RECS - 1
// (those that exist), thread tid taking pages w PREP_RECS + tid + PREP_THR i.
__device__ void prep_records(const PrepArgs& a, int tid, int w, int* s_pp, int* s_len) {
    page_prefix(a, tid, s_pp, s_len);
    const int total = s_pp[a.n];
    const int mask = (1 << a.bs_shift) - 1;
#pragma unroll
    for (int i = 0; i < PREP_RECS / PREP_THR; ++i) {
        const int gp = w * PREP_RECS + tid + PREP_THR * i;
        if (gp >= total) break;
        int lo = 0, hi = a.n - 1;  // the request of page gp: the largest b with s_pp[b] <= gp
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_pp[mid] <= gp) lo = mid; else hi = mid - 1;
        }
        const int b = lo, k = gp - s_pp[b], L = s_len[b];
        const int blk = a.bt[(int64_t)b * a.bt_s0 + (int64_t)(k >> a.bs_shift) * a.bt_s1];
        PageRec r;
        r.addr = (uint64_t)(uintptr_t)a.cache + (uint64_t)((int64_t)blk * a.c_s0 +
                                                           (int64_t)((k & mask) * TILE_TOK) * a.c_s1);
        r.k = k;
        r.bits = pr_bits(b, min(TILE_TOK, L - TILE_TOK * k), TILE_TOK * (k + 1) >= L);
        a.pages[gp] = r;
    }
}

// Workgroup 1 of prep: the wave plan. Per wave (PLAN_STRIDE ints) [0] its tiles, [1] its
// heads, [2] its heads with tiles, [3] whether every head of it has at most 4 tiles,
// [8 + s] the tile of slot s, [32 + k], [40 + k], [48 + k] head k's query head, first slot
// and tile count, [PW_SLOTS + s] the slot words; then one int, 1 if the heads fit the
// waves (every wave at most MAX_SLOTS tiles).
__device__ void prep_plan(const PrepArgs& a, const TileTable& tt, int tid) {
    __shared__ int s_byp[MAX_H];   // query head at each position of the size order
    __shared__ int s_load[NWAVE];  // tiles per decode wave
    __shared__ int s_plan[NWAVE * PLAN_STRIDE + 1];
    const int lane = tid & 63, wave = tid >> 6;
    // Heads by decreasing tile count (ties: lower head first): lane h of wave 0 counts
    // the heads before head h (every head's count read at once, four per LDS read).
    if (wave == 0) {
        const int mine = lane < a.Hq ? tt.hn[lane] : 0;
        int4 hv[MAX_H / 4];
#pragma unroll
        for (int g = 0; g < MAX_H / 4; ++g) hv[g] = ((const int4*)tt.hn)[g];
        int pos = 0;
#pragma unroll
        for (int g = 0; g < MAX_H / 4; ++g) {
            const int e[4] = {hv[g].x, hv[g].y, hv[g].z, hv[g].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int h = 4 * g + j;
                pos += h < a.Hq && (e[j] > mine || (e[j] == mine && h < lane));
            }
        }
        if (lane < a.Hq) s_byp[pos] = lane;
    }
    for (int i = tid; i < NWAVE * PLAN_STRIDE + 1; i += PREP_THR) s_plan[i] = 0;
    if (tid < NWAVE) s_load[tid] = 0;
    __syncthreads();

    // Wave plan, in wave 0 with lane p holding the head at position p of the size order.
    // Heads are dealt to the 8 waves in snake order (0..7, 7..0, 0..7, ...), so every
    // wave takes ceil(Hq / 8) or fewer heads (one head per 16-lane row of the softmax)
    // and the big heads pair with small ones; then swaps between the most loaded wave
    // and another lower the maximum while they can.
    if (wave == 0) {
        const bool act = lane < a.Hq;
        const int head = act ? s_byp[lane] : 0;
        const int hsz = act ? tt.hn[head] : 0;
        const int hfirst = act ? tt.hf[head] : 0;
        const int col = lane % NWAVE;
        int hwave = act ? (((lane / NWAVE) & 1) ? NWAVE - 1 - col : col) : -1;
        if (act) atomicAdd(&s_load[hwave], hsz);
        int load = lane < NWAVE ? s_load[lane] : 0;  // lane w < 8: wave w's tiles
        const int target = (a.TT + NWAVE - 1) / NWAVE;
        for (int it = 0; it < 64; ++it) {
            const int kmax = lanes8_max(lane < NWAVE ? (load << 8) | lane : -1);  // most loaded wave A
            const int A = kmax & 255, la = kmax >> 8;
            if (la <= target) break;
            // Candidate swaps: a head ha of A with this lane's head hb of another wave B.
            const int lb = __builtin_amdgcn_ds_bpermute(max(hwave, 0) * 4, load);  // load of hb's wave
            uint64_t inA = __builtin_amdgcn_ballot_w64(act && hwave == A);
            int best = 0x7fffffff;
            while (inA) {
                const int ha = __builtin_ctzll(inA);
                inA &= inA - 1;
                const int d = __builtin_amdgcn_readlane(hsz, ha) - hsz;
                if (act && hwave != A && d > 0 && lb + d < la)
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
        // Each head's place in its wave's plan, from its wave's heads in lane (= size)
        // order: k = the heads before it, sl = their tiles, nfb = those of them with
        // tiles; over its whole wave: nfh heads with tiles, the largest head mxh (the
        // first). Lane w < 8 also takes wave w's heads, heads with tiles, largest head.
        // The counts run as inclusive lane scans (Hq <= 32 lanes) of 8-bit fields, wave w
        // at bits 8 (w & 3) of word w >> 2 (a wave's tiles are at most MAX_TT < 256).
        const int wv = act ? hwave : 0;
        const uint32_t one = act ? 1u << (8 * (wv & 3)) : 0u;
        uint32_t c0 = wv < 4 ? one : 0u, c1 = wv < 4 ? 0u : one;  // heads
        uint32_t s0 = c0 * (uint32_t)hsz, s1 = c1 * (uint32_t)hsz;  // their tiles
        uint32_t f0 = hsz > 0 ? c0 : 0u, f1 = hsz > 0 ? c1 : 0u;    // heads with tiles
        scan32(c0); scan32(c1);
        scan32(s0); scan32(s1);
        scan32(f0); scan32(f1);
        auto fld = [](uint32_t x0, uint32_t x1, int w) -> int {
            return (int)(((w < 4 ? x0 : x1) >> (8 * (w & 3))) & 255u);
        };
        // The last head's lane holds every wave's totals.
        const uint32_t tc0 = __builtin_amdgcn_readlane(c0, a.Hq - 1), tc1 = __builtin_amdgcn_readlane(c1, a.Hq - 1);
        const uint32_t tf0 = __builtin_amdgcn_readlane(f0, a.Hq - 1), tf1 = __builtin_amdgcn_readlane(f1, a.Hq - 1);
        const int k = fld(c0, c1, wv) - 1, sl = fld(s0, s1, wv) - hsz, nfb = fld(f0, f1, wv) - (hsz > 0 ? 1 : 0);
        const int nfh = fld(tf0, tf1, wv);
        const int nhw = fld(tc0, tc1, lane & 7), nfw = fld(tf0, tf1, lane & 7);
        int mxh = 0, mxw = 0;  // a wave's largest head is its first
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
            const uint64_t bw = __builtin_amdgcn_ballot_w64(act && hwave == w);
            const int big = bw ? __builtin_amdgcn_readlane(hsz, (int)__builtin_ctzll(bw)) : 0;
            if (act && hwave == w) mxh = big;
            if (lane == w) mxw = big;
        }
        const int nnb = sl - nfb;  // tiles past their first of the heads before this one
        if (act && ok) {
            int* pw = s_plan + hwave * PLAN_STRIDE;
            pw[32 + k] = head;
            pw[40 + k] = sl;
            pw[48 + k] = hsz;
            int wd[MAX_SLOTS];  // the head's tile words, read at once (hsz <= MAX_SLOTS: the plan fits)
#pragma unroll
            for (int j = 0; j < MAX_SLOTS; ++j) wd[j] = tt.word[min(hfirst + j, MAX_TT - 1)];
#pragma unroll
            for (int j = 0; j < MAX_SLOTS; ++j) {
                if (j < hsz) {
                    pw[8 + sl + j] = hfirst + j;
                    // The decode kernel's slot order: plan order, or for the 3.2-bit kernel the
                    // heads' first tiles first (the ones with outlier ranks), then the rest.
                    const int ks = a.t_head ? (j == 0 ? nfb : nfh + nnb + j - 1) : sl + j;
                    const int row = mxh <= 4 ? 4 * k + j : sl + j;  // the slot's partial-logit row
                    pw[PW_SLOTS + ks] = slot_word(wd[j], row, k, hfirst + j);
                }
            }
        }
        if (lane < NWAVE) {
            int* pw = s_plan + lane * PLAN_STRIDE;
            pw[0] = ok ? load : 0;
            pw[1] = ok ? nhw : 0;
            pw[2] = ok ? nfw : 0;
            pw[3] = mxw <= 4;
        }
        // Slots past each wave's tiles: tile 0, the spare row (lane i: slots i, i + 64 of
        // the 8 x MAX_SLOTS).
        const uint32_t spare = slot_word(tt.word[0] & SW_CODE_MASK, MAX_SLOTS, 0, 0);
        static_assert(NWAVE * MAX_SLOTS % 64 == 0, "the spare slots fill whole passes of the wave");
#pragma unroll
        for (int i = 0; i < NWAVE * MAX_SLOTS; i += 64) {
            const int w = (i + lane) / MAX_SLOTS, s2 = (i + lane) % MAX_SLOTS;
            const int lw = __shfl(load, w, 64);
            if (s2 >= (ok ? lw : 0)) s_plan[w * PLAN_STRIDE + PW_SLOTS + s2] = (int)spare;
        }
        if (lane == 0) s_plan[NWAVE * PLAN_STRIDE] = ok;
    }
    __syncthreads();
    int* plan = (int*)(a.ws + a.ws_plan);
    for (int i = tid; i < NWAVE * PLAN_STRIDE + 1; i += PREP_THR) plan[i] = s_plan[i];
}

// Eight consecutive elements of a DT array from element i, as raw bits (2-byte types:
// r[0]; fp32: r[0], r[1]), and their fp32 values.
template <int DT>
struct Raw8 {
    uint4 r[DT == STARKV_F32 ? 2 : 1];
};
template <int DT>
__device__ __forceinline__ Raw8<DT> raw8(const void* p, int64_t i) {
    Raw8<DT> v;
    if constexpr (DT == STARKV_F32) {
        const uint4* s = (const uint4*)((const float*)p + i);
        v.r[0] = s[0];
        v.r[1] = s[1];
    } else {
        v.r[0] = *(const uint4*)((const uint16_t*)p + i);
    }
    return v;
}
template <int DT>
__device__ __forceinline__ void raw8_f(const Raw8<DT>& v, float* o) {
    if constexpr (DT == STARKV_F32) {
        const uint32_t w[8] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w, v.r[1].x, v.r[1].y, v.r[1].z, v.r[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __uint_as_float(w[e]);
    } else {
        const uint32_t w[4] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (DT == STARKV_BF16) {
                o[2 * k] = __uint_as_float(w[k] << 16);
                o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            } else {
                const half2_t h = __builtin_bit_cast(half2_t, w[k]);
                o[2 * k] = (float)h[0];
                o[2 * k + 1] = (float)h[1];
            }
        }
    }
}

// Fold workgroups of prep: AB[b][t][ks][lane] = 8 fp16 of tile row m = lane & 15,
// columns 32 ks + 8 (lane >> 4) .. +8, scaled by scale*log2(e); rows past the head's
// rank are zero (paged_decode.py:79-81 masks them). Row m holds rank m of the tile, or,
// for the 3.2-bit cache, rank 2 (m >> 2) + ((m >> 1) & 1) + 8 (m & 1), scaled by 1/16
// when m & 2: then the z values a lane receives (rows 4g .. 4g+3) are ranks 2g, 2g+8,
// 2g+1, 2g+9, the low and high nibbles of bytes g and g+4 of the tile's 8 code bytes
// (the high nibbles are read as 16 n). Thread (tile, k2, lane) reads its two k_up
// granules once and folds them with the query of each of its requests; every load is
// issued before the first conversion, so their latencies overlap.
template <int QT, int UT>
__device__ void prep_fold(const PrepArgs& a, const TileTable& tt, int tid, int bid) {
    const int tp = bid % a.tile_pairs, b0 = (bid / a.tile_pairs) * PREP_REQ;
    const int t = 2 * tp + (tid >> 7), k2 = (tid >> 6) & 1, lane = tid & 63;
    if (t >= a.TT) return;
    const bool perm = a.t_head != nullptr;
    const int m = lane & 15, lg = lane >> 4;
    const int rr = perm ? 2 * (m >> 2) + ((m >> 1) & 1) + 8 * (m & 1) : m;
    const int c0 = 32 * k2 + 8 * lg;
    const int h = tt.head[t];
    const float s = rr < tt.valid[t] ? (perm && (m & 2) ? a.sc * 0.0625f : a.sc) : 0.f;
    const int64_t ur = (int64_t)(tt.row[t] + rr) * a.ku_s0;
    const Raw8<UT> ru0 = raw8<UT>(a.k_up, ur + c0), ru1 = raw8<UT>(a.k_up, ur + c0 + 64);
    Raw8<QT> rq0[PREP_REQ], rq1[PREP_REQ];
#pragma unroll
    for (int i = 0; i < PREP_REQ; ++i) {
        const int b = min(b0 + i, a.n - 1);
        const int64_t qh = (int64_t)b * a.q_s0 + (int64_t)h * a.q_s1;
        rq0[i] = raw8<QT>(a.q, qh + c0);
        rq1[i] = raw8<QT>(a.q, qh + c0 + 64);
    }
    float u0[8], u1[8];
    raw8_f<UT>(ru0, u0);
    raw8_f<UT>(ru1, u1);
#pragma unroll
    for (int i = 0; i < PREP_REQ; ++i) {
        float q0[8], q1[8];
        raw8_f<QT>(rq0[i], q0);
        raw8_f<QT>(rq1[i], q1);
        half8_t x, y;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = (_Float16)((q0[e] * u0[e] + q1[e] * u1[e]) * s);
            y[e] = (_Float16)((q1[e] * u0[e] - q0[e] * u1[e]) * s);
        }
        if (b0 + i < a.n) {
            half8_t* o = (half8_t*)(a.ws + a.ws_ab + ((size_t)(b0 + i) * a.TT + t) * AB_TILE_BYTES);
            o[k2 * 64 + lane] = x;
            o[(k2 + 2) * 64 + lane] = y;
        }
    }
}

template <int QT>
__device__ void prep_fold_q(const PrepArgs& a, const TileTable& tt, int tid, int bid) {
    if (a.ku_dt == STARKV_BF16)
        prep_fold<QT, STARKV_BF16>(a, tt, tid, bid);
    else if (a.ku_dt == STARKV_F16)
        prep_fold<QT, STARKV_F16>(a, tt, tid, bid);
    else
        prep_fold<QT, STARKV_F32>(a, tt, tid, bid);
}

// Workgroup `bid` of prep's grid: 0 the prefix, 1 the plan, then the fold workgroups,
// then the record workgroups.
__device__ __forceinline__ void prep_block(const PrepArgs& a, int bid) {
    __shared__ TileTable tt;
    __shared__ int s_pp[MAX_REQ_PER_CALL + 1], s_len[MAX_REQ_PER_CALL];
    const int tid = threadIdx.x;
    if (bid == 0) {
        prep_prefix(a, tid, s_pp, s_len);
        return;
    }
    if (bid >= 2 + a.fold_wgs) {
        prep_records(a, tid, bid - 2 - a.fold_wgs, s_pp, s_len);
        return;
    }
    tile_table(a, tt, tid);
    if (bid == 1) {
        prep_plan(a, tt, tid);
    } else if (a.q_dt == STARKV_BF16) {
        prep_fold_q<STARKV_BF16>(a, tt, tid, bid - 2);
    } else if (a.q_dt == STARKV_F16) {
        prep_fold_q<STARKV_F16>(a, tt, tid, bid - 2);
    } else {
        prep_fold_q<STARKV_F32>(a, tt, tid, bid - 2);
    }
}

__global__ __launch_bounds__(PREP_THR) void prep_kernel(PrepArgs a) { prep_block(a, blockIdx.x); }

// prep with a deferred cache write's code GEMM in the same launch (the two are
// independent: prep reads the query, lengths, tables and block table, the GEMM the
// layer input and kv_down): prep's workgroups first, then the GEMM's (gx x gy x gz grid
// flattened). The write's store follows as the next launch, before the decode kernels.
static_assert(KVW_THR == PREP_THR, "the GEMM and prep workgroups share one launch");
template <int DT>
__global__ __launch_bounds__(PREP_THR) void write_prep_kernel(PrepArgs a, KvGemmParams g, int prep_wgs, int gx,
                                                              int gy) {
    const int bid = blockIdx.x;
    if (bid < prep_wgs) {
        prep_block(a, bid);
        return;
    }
    const int gb = bid - prep_wgs;
    kv_gemm_block<DT>(g, gb % gx, (gb / gx) % gy, gb / (gx * gy));
}
// The same with the direct form of the write (one or two tokens): its jobs after prep's
// workgroups.
template <int DT, int TOK, int SL>
__global__ __launch_bounds__(PREP_THR) void write_prep_direct_kernel(PrepArgs a, KvDirectParams d, int prep_wgs) {
    const int bid = blockIdx.x;
    if (bid < prep_wgs) {
        prep_block(a, bid);
        return;
    }
    kv_direct_block<DT, TOK, SL>(d, bid - prep_wgs);
}
template <int DT>
static const void* write_prep_direct_fn(int n, int slices) {
    if (slices == KVD_MAX_SLICES)
        return n == 1 ? (const void*)&write_prep_direct_kernel<DT, 1, KVD_MAX_SLICES>
                      : (const void*)&write_prep_direct_kernel<DT, 2, KVD_MAX_SLICES>;
    return (const void*)&write_prep_direct_kernel<DT, 1, 0>;  // two tokens take the direct form only at SL
}

// ---------------------------------------------------------------------------
// 3. merge: per (request, head) the partials' log-sum-exp, then the lift through
//    v_up_by_q. A workgroup takes one head and MERGE_REQ requests, one wave each, so
//    every row of v_up_by_q[h] serves MERGE_REQ outputs; a call of one or two requests
//    gives each request 4 or 2 waves, which split its partials (partial k to wave k mod
//    the waves) and add their rows before the lift. The loads come in two phases: the
//    request's partial range (with v_up_by_q[h] staged into LDS meanwhile), then the max
//    and sum of the first 64 MERGE_ML partials and the wave's first PRE partials'
//    accumulator rows together (PRE = 32 at V rank <= 64, else 16); further partials
//    follow PRE rows at a time.
// ---------------------------------------------------------------------------
constexpr int MERGE_REQ = 4;
constexpr int MERGE_THR = 64 * MERGE_REQ;
constexpr int MERGE_CB = 4;   // column blocks of 64: v_rank <= 256
constexpr int MERGE_ML = 4;   // partials' (max, sum) per lane read in the second round: 256 per request

// LDS of one merge workgroup: v_up_by_q[h] (v_rank x 128 WT), then the merged
// low-rank outputs [MERGE_REQ][v_rank] (fp32).
static size_t merge_lds_bytes(int v_rank, int w_dt) {
    return (size_t)v_rank * 128 * (w_dt == STARKV_F32 ? 4 : 2) + (size_t)MERGE_REQ * v_rank * 4;
}

template <typename WT>
__device__ __forceinline__ float lds_w(const WT* p, int i);
template <>
__device__ __forceinline__ float lds_w<uint16_t>(const uint16_t* p, int i) { return bf16_bits_to_f32(p[i]); }
template <>
__device__ __forceinline__ float lds_w<_Float16>(const _Float16* p, int i) { return (float)p[i]; }
template <>
__device__ __forceinline__ float lds_w<float>(const float* p, int i) { return p[i]; }

// CB: columns per lane (v_rank <= 64 CB); PRE partials' rows per wave in the second round.
template <typename WT, int CB>
__global__ __launch_bounds__(MERGE_THR) void merge_kernel(const uint8_t* __restrict__ ws, size_t ws_plan,
                                                          size_t ws_m, size_t ws_l, size_t ws_acc, int n, int Hq,
                                                          int v_rank, const WT* __restrict__ vup, int64_t vu_s0,
                                                          int64_t vu_s1, void* __restrict__ out, int64_t o_s0,
                                                          int64_t o_s1, int out_dt) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    WT* s_v = (WT*)s_dyn;                                     // [v_rank][128]
    float* s_o = (float*)(s_dyn + (size_t)v_rank * 128 * sizeof(WT));  // [MERGE_REQ][v_rank]
    __shared__ int s_live[MERGE_REQ];
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    // Requests per workgroup (grid.x is 1 when n < 3) and waves per request.
    const int rpw = n >= 3 ? MERGE_REQ : n, wpr = MERGE_REQ / rpw;
    const int r = (tid >> 6) / wpr, sub = (tid >> 6) % wpr;  // this wave's request and share
    const int b = blockIdx.x * MERGE_REQ + r;
    const int* hdr = (const int*)ws;
    const float* wm = (const float*)(ws + ws_m);
    const float* wl = (const float*)(ws + ws_l);
    const float* wa = (const float*)(ws + ws_acc);

    // Load phase 1: request b's tokens [pb, pe) in the concatenation, hence its partial slots
    // k_lo + k + b, k < nk (S tokens per decode workgroup). No tokens: softmax over an
    // empty row (NaN, as the reference). No wave plan (a head assignment that does not
    // fit): NaN as well, never a silent wrong result.
    const int S = hdr[0];
    const bool planned = ((const int*)(ws + ws_plan))[NWAVE * PLAN_STRIDE] != 0;
    const int pb = b < n ? hdr[1 + b] : 0, pe = b < n ? hdr[2 + b] : 0;
    {
        // v_up_by_q[h] into LDS, 8 granules (16 bytes) per thread in flight at a time.
        constexpr int GPR = 128 * (int)sizeof(WT) / 16;  // granules per row
        constexpr int BATCH = 8;
        const uint8_t* vh = (const uint8_t*)(vup + (int64_t)h * vu_s0);
        const int total = v_rank * GPR;
        for (int base = 0; base < total; base += BATCH * MERGE_THR) {
            uint4 g[BATCH];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int i = min(base + u * MERGE_THR + tid, total - 1), c = i / GPR;  // no branch: loads overlap
                g[u] = *(const uint4*)(vh + (int64_t)c * vu_s1 * (int64_t)sizeof(WT) + 16 * (i - c * GPR));
            }
#pragma unroll
            for (int u = 0; u < BATCH; ++u)  // past the end: granule total - 1 again, same bytes
                ((uint4*)s_dyn)[min(base + u * MERGE_THR + tid, total - 1)] = g[u];
        }
    }
    const bool live = b < n && pe > pb && S > 0 && planned;
    const int k_lo = live ? pb / S : 0, nk = live ? (pe - 1) / S - k_lo + 1 : 0;
    const int64_t s0 = (int64_t)(k_lo + b) * Hq + h;  // slot index of partial k: s0 + k * Hq

    // Load phase 2: partials k = lane + 64 j's max and sum (j < MERGE_ML), and lane's columns
    // c = lane + 64 j of the wave's first PRE partials (k = sub + wpr i).
    constexpr int PRE = CB == 1 ? 32 : 16;
    float mk[MERGE_ML], lk[MERGE_ML];
#pragma unroll
    for (int j = 0; j < MERGE_ML; ++j) {
        const int k = lane + 64 * j;
        mk[j] = k < nk ? wm[s0 + (int64_t)k * Hq] : -INFINITY;
        lk[j] = k < nk ? wl[s0 + (int64_t)k * Hq] : 0.f;
    }
    float pre[PRE][CB];
#pragma unroll
    for (int i = 0; i < PRE; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int c = lane + 64 * j, k = sub + wpr * i;
            pre[i][j] = k < nk && c < v_rank ? wa[(s0 + (int64_t)k * Hq) * v_rank + c] : 0.f;
        }
    float M = mk[0];
#pragma unroll
    for (int j = 1; j < MERGE_ML; ++j) M = fmaxf(M, mk[j]);
    for (int k = lane + 64 * MERGE_ML; k < nk; k += 64) M = fmaxf(M, wm[s0 + (int64_t)k * Hq]);
    M = wave_max(M);
    float wk[MERGE_ML];  // weight of partial lane + 64 j
    float l = 0.f;
#pragma unroll
    for (int j = 0; j < MERGE_ML; ++j) {
        wk[j] = lane + 64 * j < nk ? exp2f(mk[j] - M) : 0.f;
        l = fmaf(lk[j], wk[j], l);
    }
    for (int k = lane + 64 * MERGE_ML; k < nk; k += 64) {
        const int64_t sl = s0 + (int64_t)k * Hq;
        l += wl[sl] * exp2f(wm[sl] - M);
    }
    l = wave_sum(l);
    // Weight of partial k (wave-uniform), read across lanes (every lane active here).
    static_assert(MERGE_ML == 4, "the weights in registers are wk[0 .. 3]");
    const float wk0 = wk[0], wk1 = wk[1], wk2 = wk[2], wk3 = wk[3];
    auto weight = [=](int k) -> float {
        if (k < 64 * MERGE_ML) {
            const int j = k >> 6;
            const float x = j == 0 ? wk0 : j == 1 ? wk1 : j == 2 ? wk2 : wk3;
            return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k & 63));
        }
        return exp2f(wm[s0 + (int64_t)k * Hq] - M);
    };
    float acc[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[j] = 0.f;
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
        const int k = sub + wpr * i;  // wave-uniform
        if (k >= nk) break;
        const float w = weight(k);
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[j] = fmaf(pre[i][j], w, acc[j]);
    }
    // Requests spread over more than wpr PRE workgroups: PRE of the wave's partials' rows
    // in flight at a time (columns past v_rank read column 0 and are never stored).
    for (int i0 = PRE; sub + wpr * i0 < nk; i0 += PRE) {
        float v[PRE][CB];
#pragma unroll
        for (int u = 0; u < PRE; ++u) {
            const int64_t sl = s0 + (int64_t)min(sub + wpr * (i0 + u), nk - 1) * Hq;
#pragma unroll
            for (int j = 0; j < CB; ++j) {
                const int c = lane + 64 * j;
                v[u][j] = wa[sl * v_rank + (c < v_rank ? c : 0)];
            }
        }
#pragma unroll
        for (int u = 0; u < PRE; ++u) {
            const int k = sub + wpr * (i0 + u);
            if (k >= nk) break;
            const float w = weight(k);
#pragma unroll
            for (int j = 0; j < CB; ++j) acc[j] = fmaf(v[u][j], w, acc[j]);
        }
    }
    // Row (tid >> 6) of s_o: this wave's share of request r, scaled; a request's wpr rows
    // (rows r wpr + s) are added into row r before the lift.
    const float inv = 1.f / l;
#pragma unroll
    for (int j = 0; j < CB; ++j)
        if (lane + 64 * j < v_rank) s_o[(tid >> 6) * v_rank + lane + 64 * j] = acc[j] * inv;
    if (lane == 0 && sub == 0) s_live[r] = live;
    __syncthreads();

    if (wpr > 1) {  // rows r wpr .. r wpr + wpr - 1 into row r (r < rpw), column tid
        float x0 = 0.f, x1 = 0.f;
        if (tid < v_rank) {
            for (int s2 = 0; s2 < wpr; ++s2) {
                x0 += s_o[s2 * v_rank + tid];
                if (rpw == 2) x1 += s_o[(wpr + s2) * v_rank + tid];
            }
        }
        __syncthreads();
        if (tid < v_rank) {
            s_o[tid] = x0;
            if (rpw == 2) s_o[v_rank + tid] = x1;
        }
        __syncthreads();
    }

    // The lift through v_up_by_q[h]: thread (d, request pair) takes two requests' column d.
    const int d = tid & 127, r0 = 2 * (tid >> 7);
    float o0 = 0.f, o1 = 0.f;
#pragma unroll 8
    for (int c = 0; c < v_rank; ++c) {
        const float v = lds_w<WT>(s_v, c * 128 + d);
        o0 = fmaf(s_o[r0 * v_rank + c], v, o0);
        o1 = fmaf(s_o[(r0 + 1) * v_rank + c], v, o1);
    }
    const int bb = blockIdx.x * MERGE_REQ + r0;
    if (bb < n) store_f(out, (int64_t)bb * o_s0 + (int64_t)h * o_s1 + d, out_dt, s_live[r0] ? o0 : __builtin_nanf(""));
    if (bb + 1 < n)
        store_f(out, (int64_t)(bb + 1) * o_s0 + (int64_t)h * o_s1 + d, out_dt,
                s_live[r0 + 1] ? o1 : __builtin_nanf(""));
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
int device_cus() {
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

// tok_per_wg: tokens per workgroup the split aims for (at most the device's CUs
// workgroups). 64 for the one-pass kernels and the logits pass of two-pass calls, whose
// partials are small, so that a short batch (one request of 4096 tokens) still spreads
// over many CUs; PV_TOK for the P @ V pass of two-pass calls (pv_ratio).
static int grid_for(int n, int max_seq_len, int tok_per_wg = 256) {
    const int64_t tokens = (int64_t)n * (int64_t)(max_seq_len > 0 ? max_seq_len : 1);
    int64_t want = (tokens + tok_per_wg - 1) / tok_per_wg;
    // Each request a workgroup moves on to costs a reload of that request's folded query
    // tiles (about as long as 2-3 pages), so short requests get a workgroup each where the
    // device has one to spare.
    if (want < n) want = n;
    const int cus = device_cus();
    if (want > cus) want = cus;
    return want < 1 ? 1 : (int)want;
}

// Two-pass calls: the P @ V pass runs over ranges of R consecutive logits-pass ranges. Its
// fp32 partial accumulators of H x v_rank per workgroup and request cost about as much
// traffic as the V codes they sum when a workgroup has few pages, while the logits pass's
// partials are two floats per head: with few requests the logits pass takes every CU and
// the P @ V pass fewer, longer ranges in column windows side by side. R = the logits grid
// over the grid at PV_TOK tokens per workgroup, rounded (1 to 4). One request of 16419
// tokens at V rank 1280 / 1290 (config 4 at concurrency 1), P @ V + merge: bf16 36.7 us at
// R = 2, 37.6 at R = 1; 3.2-bit 34.6 us at R = 2, 35.4 at R = 1, 39.3 at R = 4 (a P @ V
// page costs about the same at a quarter of the columns). Two such requests: R = 1 for
// both, the fastest.
constexpr int PV_TOK = 128;
static int pv_ratio(int fmt, int n, int max_seq_len, int grid) {
    (void)fmt;
    const int gp = grid_for(n, max_seq_len, PV_TOK);
    return std::max(1, std::min(4, (grid + gp / 2) / gp));
}

// Optional timing for benchmarks: when armed, each call records a HIP event pair on the
// caller's stream, around its decode kernels (mode 0: the one-pass kernel, or the logits
// and P @ V passes) or around the whole call (mode 1: prep to merge).
struct DecodeProfile {
    bool on = false;
    int mode = 0;
    int used = 0;
    std::vector<hipEvent_t> ev;
    std::vector<double> ms;  // per-call durations of the last profile_end
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
    int head0, code0;
    const void* vup; int64_t vu_s0, vu_s1; int vu_dt; int v_rank;
    const void* cs; int64_t cs_s0; int cs_dt;
    float scale;
    void* out; int64_t o_s0, o_s1; int out_dt;
    void* ws; size_t ws_bytes;
    int grid;
};

template <typename WT, int CB>
static int launch_merge_cb(dim3 grid, size_t lds, hipStream_t stream, const DecodeParams& p, const WsLayout& wl,
                           const CommonArgs& a) {
    static size_t lds_allowed = 65536;  // per function: raised as larger v_rank need it (at most 132 KB)
    if (lds > lds_allowed) {
        SKV_HIP(hipFuncSetAttribute((const void*)merge_kernel<WT, CB>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds));
        lds_allowed = lds;
    }
    hipLaunchKernelGGL((merge_kernel<WT, CB>), grid, dim3(MERGE_THR), lds, stream, (const uint8_t*)p.ws, wl.plan, wl.m,
                       wl.l, wl.acc, a.n, a.Hq, a.v_rank, (const WT*)a.vup, a.vu_s0, a.vu_s1, a.out, a.o_s0, a.o_s1,
                       a.out_dt);
    SKV_HIP(hipGetLastError());
    return STARKV_OK;
}

// One column per lane up to V rank 64 (the partials' rows of 32 partials per wave in flight
// together), else four.
template <typename WT>
static int launch_merge(dim3 grid, size_t lds, hipStream_t stream, const DecodeParams& p, const WsLayout& wl,
                        const CommonArgs& a) {
    return a.v_rank <= 64 ? launch_merge_cb<WT, 1>(grid, lds, stream, p, wl, a)
                          : launch_merge_cb<WT, MERGE_CB>(grid, lds, stream, p, wl, a);
}

// Which decode form runs: 0 = the one-pass kernels where the shape fits them, else the
// two-pass form; 1 = one-pass only (shapes it cannot take are refused); 2 = two-pass
// always. Set by starkv_decode_set_path (tests and benchmarks compare the two).
static int g_path = 0;

// Whether the one-pass kernel takes a layer of this shape.
// TT: the call's rank tiles over its query heads (the tiles per wave the kernel must hold
// decide whether a one-pass instantiation without scratch spills exists).
static bool one_pass_fits(int fmt, int k_width, int v_rank, int row_bytes, int v_nout, int TT) {
    if (fmt == FMT_Q4) {
        const int qnb = quant_v_blocks(v_rank, v_nout);
        return qnb > 0 && quant_copies(row_bytes) > 0 && quant_lds_bytes(row_bytes, qnb) <= quant_lds_limit() &&
               quant_mtv(TT, qnb, row_bytes) > 0;
    }
    const int nb = (v_rank + 63) / 64;
    return nb <= 4 && lowrank_copies(k_width, nb) > 0 && lowrank_mtv(TT, nb) > 0;
}

static bool use_two_pass(int fmt, int k_width, int v_rank, int row_bytes, int v_nout, int TT) {
    return g_path == 2 || (g_path == 0 && !one_pass_fits(fmt, k_width, v_rank, row_bytes, v_nout, TT));
}

// Host restatement of the wave plan that workgroup 1 of prep_kernel builds
// (prep_plan): query heads sorted by decreasing rank tiles (ties: lower head first),
// dealt to the 8 decode waves in snake order, then the swap that lowers the most loaded
// wave the most, while one does. True if every wave ends with at most MAX_SLOTS tiles,
// which is when the decode kernels run the layer (otherwise they return NaN rows).
static bool plan_fits(const int* tiles, int Hq, int TT) {
    if (Hq < 1 || Hq > MAX_H || TT < 1 || TT > MAX_TT) return false;
    int head_at[MAX_H], hsz[MAX_H], hwave[MAX_H], load[NWAVE] = {0};
    for (int h = 0; h < Hq; ++h) {
        int pos = 0;
        for (int k = 0; k < Hq; ++k) pos += tiles[k] > tiles[h] || (tiles[k] == tiles[h] && k < h);
        head_at[pos] = h;
    }
    for (int p = 0; p < Hq; ++p) {
        hsz[p] = tiles[head_at[p]];
        const int col = p % NWAVE;
        hwave[p] = ((p / NWAVE) & 1) ? NWAVE - 1 - col : col;
        load[hwave[p]] += hsz[p];
    }
    const int target = (TT + NWAVE - 1) / NWAVE;
    for (int it = 0; it < 64; ++it) {
        int A = 0;
        for (int w = 1; w < NWAVE; ++w)
            if (load[w] >= load[A]) A = w;  // the most loaded wave, ties to the higher index
        const int la = load[A];
        if (la <= target) break;
        int best = 0x7fffffff;
        for (int ha = 0; ha < Hq; ++ha) {
            if (hwave[ha] != A) continue;
            for (int hb = 0; hb < Hq; ++hb) {
                if (hwave[hb] == A) continue;
                const int d = hsz[ha] - hsz[hb], lb = load[hwave[hb]];
                if (d > 0 && lb + d < la) best = std::min(best, (std::max(la - d, lb + d) << 16) | (ha << 8) | hb);
            }
        }
        if (best == 0x7fffffff) break;
        const int ha = (best >> 8) & 255, hb = best & 255, B = hwave[hb], d = hsz[ha] - hsz[hb];
        hwave[ha] = B;
        hwave[hb] = A;
        load[A] -= d;
        load[B] += d;
    }
    for (int w = 0; w < NWAVE; ++w)
        if (load[w] > MAX_SLOTS) return false;
    return true;
}

static int lcap_of(int max_seq_len) { return (max_seq_len + TILE_TOK - 1) / TILE_TOK * TILE_TOK; }

// QuantRow (paged_quant.py:71-111) offsets of a 3.2-bit row.
struct QRow {
    int v_rank, v_nout, v_nbo, ks_off, vs_off, vq_off, v_bytes, nbytes;
};
static QRow qrow(int k_width, int num_heads, int v_rank) {
    QRow r;
    r.v_rank = v_rank;
    r.v_nout = (int)(0.2 * (double)v_rank);
    r.v_nbo = (r.v_nout + 1) / 2;
    r.ks_off = k_width / 2;
    r.vs_off = r.ks_off + 4 * num_heads;
    r.vq_off = r.vs_off + 4;
    r.v_bytes = r.v_nbo + (v_rank - r.v_nout + 1) / 2;
    r.nbytes = (r.vq_off + r.v_bytes + 15) / 16 * 16;
    return r;
}

// A 3.2-bit call over query heads [head0, head0 + heads) of a layer whose rows are
// QuantRow(row_k_width, row_heads, v_rank), the heads' K lanes starting at lane0 (a
// multiple of 16). Its cache pointer is advanced to the 16-byte granule `base` holding
// the group's first K nibble byte; every offset below is relative to it. The copies of
// a page take the bytes from there to the row's end (one pass) or to the group's last K
// scale (the logits pass of two-pass calls).
struct QGroup {
    QRow row;       // the layer's row
    int base;       // bytes the cache pointer advances
    int code0;      // code tile (8 bytes) of the group's first tile, from base
    int ks_off, vs_off, vq_off;
    int extent;     // bytes from base to the row's end (a multiple of 16)
    int k_extent;   // bytes from base through the group's K scales, rounded up to 16
};
static QGroup qgroup(int row_k_width, int row_heads, int v_rank, int head0, int heads, int lane0) {
    QGroup g;
    g.row = qrow(row_k_width, row_heads, v_rank);
    const int kb = lane0 / 2;
    g.base = kb & ~15;
    g.code0 = (kb - g.base) / 8;
    g.ks_off = g.row.ks_off + 4 * head0 - g.base;
    g.vs_off = g.row.vs_off - g.base;
    g.vq_off = g.row.vq_off - g.base;
    g.extent = g.row.nbytes - g.base;
    g.k_extent = (g.ks_off + 4 * heads + 15) / 16 * 16;
    return g;
}

static bool qgroup_args_ok(int row_k_width, int row_heads, int v_rank, int head0, int heads, int lane0,
                           int k_width) {
    return row_k_width >= 16 && row_k_width % 16 == 0 && row_heads >= 1 && v_rank >= 1 && head0 >= 0 &&
           heads >= 1 && head0 + heads <= row_heads && lane0 >= 0 && lane0 % 16 == 0 && k_width >= 16 &&
           k_width % 16 == 0 && lane0 + k_width <= row_k_width;
}

// Whether a 3.2-bit call over this group takes the two-pass form.
static bool qgroup_two_pass(const QGroup& g, int k_width) {
    return use_two_pass(FMT_Q4, 0, g.row.v_rank, g.extent, g.row.v_nout, k_width / 16);
}

// Whether one 3.2-bit call takes query heads [h0, h1) of an MHA layer of H heads with K
// ranks `ranks`: at most 32 heads and 96 rank tiles, a wave plan in which every wave
// holds at most 16 tiles, and pages (from the group's first K byte) that fit in LDS.
static bool quant_group_fits(const int32_t* ranks, int H, int v_rank, int h0, int h1) {
    const int heads = h1 - h0;
    if (heads < 1 || heads > MAX_H || h0 < 0 || h1 > H || v_rank < 1 || v_rank > MAX_V_RANK_TWO_PASS) return false;
    int tiles[MAX_H];
    int TT = 0, lane0 = 0, kw = 0, row_kw = 0;
    for (int h = 0; h < H; ++h) {
        if (ranks[h] < 0 || ranks[h] > 16 * MAX_TT) return false;
        const int w = (ranks[h] + 15) / 16 * 16;
        if (h < h0) lane0 += w;
        if (h >= h0 && h < h1) {
            kw += w;
            tiles[h - h0] = w / 16;
            TT += w / 16;
        }
        row_kw += w;
    }
    if (TT < 1 || TT > MAX_TT || !plan_fits(tiles, heads, TT)) return false;
    const QGroup g = qgroup(row_kw, H, v_rank, h0, heads, lane0);
    if (!qgroup_two_pass(g, kw)) return true;
    return quant_copies(g.k_extent) > 0 && quant_lds_bytes(g.k_extent, 0) <= quant_lds_limit() &&
           pv_fits(FMT_Q4, kw, v_rank, g.vs_off, g.vq_off, g.row.v_nout, g.row.v_bytes);
}

// Whether one bf16/fp16 call takes KV heads with K ranks ranks[0 .. hkv) and `per` query
// heads each: the call reads their K lanes and the V codes.
static bool codes_group_fits(int cache_kind, int per, const int32_t* ranks, int hkv, int v_rank) {
    const int Hq = per * hkv;
    if (Hq < 1 || Hq > MAX_H || v_rank < 1 || v_rank > MAX_V_RANK_TWO_PASS) return false;
    int tiles[MAX_H];
    int TT = 0, k_width = 0;
    for (int kv = 0; kv < hkv; ++kv) {
        const int r = ranks[kv];
        if (r < 0 || r > 16 * MAX_TT) return false;
        k_width += (r + 15) / 16 * 16;
        for (int j = 0; j < per; ++j) tiles[kv * per + j] = (r + 15) / 16;
    }
    for (int h = 0; h < Hq; ++h) TT += tiles[h];
    if (TT < 1 || TT > MAX_TT || !plan_fits(tiles, Hq, TT)) return false;
    const int fmt = cache_kind == STARKV_F16 ? FMT_F16 : FMT_BF16;
    if (!use_two_pass(fmt, k_width, v_rank, (k_width + v_rank) * 2, 0, TT)) return true;
    return lowrank_copies(k_width, 0) > 0 && pv_fits(fmt, k_width, v_rank, 0, 0, 0, 0);
}

static int decode_common_body(DecodeParams& p, const CommonArgs& a, int fmt, int row_bytes, int TT,
                              hipStream_t stream);

// A call that fails its checks leaves no deferred write behind: it is launched on its own.
static int decode_common(DecodeParams& p, const CommonArgs& a, int fmt, int row_bytes, int TT, hipStream_t stream) {
    const int rc = decode_common_body(p, a, fmt, row_bytes, TT, stream);
    if (rc != STARKV_OK) flush_pending_write();
    return rc;
}

static int decode_common_body(DecodeParams& p, const CommonArgs& a, int fmt, int row_bytes, int TT,
                              hipStream_t stream) {
    SKV_CHECK(a.n >= 1 && a.n <= MAX_REQ_PER_CALL, "decode: n=%d requests (1..%d per call)", a.n, MAX_REQ_PER_CALL);
    SKV_CHECK(a.Hq >= 1 && a.Hq <= MAX_H, "decode: num_heads=%d (1..%d)", a.Hq, MAX_H);
    SKV_CHECK(a.max_seq_len >= 1, "decode: max_seq_len must be >= 1");
    SKV_CHECK(a.v_rank >= 1, "decode: v_rank must be >= 1");
    SKV_CHECK(a.grid >= 1, "decode: grid must be >= 1");
    SKV_CHECK(TT >= 1 && TT <= MAX_TT, "decode: %d rank tiles (1..%d: k_width x heads per kv head <= %d)", TT,
              MAX_TT, MAX_TT * 16);
    const bool two = use_two_pass(fmt, p.k_width, a.v_rank, row_bytes, p.v_nout, TT);
    p.vp.n = 0;
    const int lcap = two ? lcap_of(a.max_seq_len) : 0;
    const int pv_r = two ? pv_ratio(fmt, a.n, a.max_seq_len, a.grid) : 1;
    SKV_CHECK(a.max_seq_len <= (1 << 24), "decode: max_seq_len %d > 2^24", a.max_seq_len);
    const WsLayout wl = ws_layout(a.n, a.Hq, TT, a.v_rank, a.grid, lcap, pv_r, pages_of(a.max_seq_len));
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
    SKV_CHECK(a.q_dt >= STARKV_F32 && a.q_dt <= STARKV_BF16 && a.w_dt >= STARKV_F32 && a.w_dt <= STARKV_BF16 &&
                  a.vu_dt >= STARKV_F32 && a.vu_dt <= STARKV_BF16 && a.out_dt >= STARKV_F32 &&
                  a.out_dt <= STARKV_BF16,
              "decode: query, k_up, v_up_by_q and output dtypes must be bf16, fp16 or fp32");
    SKV_CHECK(a.cs_dt == STARKV_F16, "decode: cos_sin must be fp16 (convert the table once; it is exact for bf16)");
    SKV_CHECK(a.cs_s0 % 8 == 0 && a.cs_s0 >= 128 && a.cs_s0 * 2 * TILE_TOK < ((int64_t)1 << 31) &&
                  ((uintptr_t)a.cs % 16) == 0,
              "decode: cos_sin rows must be 16-byte aligned with stride >= 128");
    SKV_CHECK(a.q_s1 % 8 == 0 && a.q_s0 % 8 == 0 && ((uintptr_t)a.q % 16) == 0,
              "decode: query rows must be 16-byte aligned (strides multiples of 8)");
    SKV_CHECK(a.ku_s0 % 8 == 0 && ((uintptr_t)a.k_up % 16) == 0, "decode: k_up rows must be 16-byte aligned");
    const int nb = (a.v_rank + 63) / 64;
    SKV_CHECK(two || one_pass_fits(fmt, p.k_width, a.v_rank, row_bytes, p.v_nout, TT),
              "decode: v_rank %d does not fit the one-pass decode (the two-pass form is switched off)", a.v_rank);
    SKV_CHECK(!two || a.v_rank <= MAX_V_RANK_TWO_PASS, "decode: v_rank %d > %d", a.v_rank, MAX_V_RANK_TWO_PASS);
    const int wsz = a.vu_dt == STARKV_F32 ? 4 : 2;
    SKV_CHECK(((uintptr_t)a.vup % 16) == 0 && (a.vu_s0 * wsz) % 16 == 0 && (a.vu_s1 * wsz) % 16 == 0,
              "decode: v_up_by_q rows must be 16-byte aligned");

    p.bt = a.bt; p.bt_s0 = (int)a.bt_s0; p.bt_s1 = (int)a.bt_s1;
    p.n = a.n; p.Hq = a.Hq; p.TT = TT; p.v_rank = a.v_rank;
    p.cs = (const uint8_t*)a.cs; p.cs_s0b = (int)(a.cs_s0 * 2);
    p.row_g = row_bytes / 16;
    int qnb = 0;
    if (two) {
        // The logits pass copies only what the K side reads: the cos/sin rows and the K
        // codes (bf16/fp16), or the K nibbles and scales (3.2-bit).
        SKV_CHECK((int64_t)a.n * a.Hq * lcap < ((int64_t)1 << 31), "decode: %d x %d x %d logits exceed 2^31", a.n,
                  a.Hq, lcap);
        SKV_CHECK(pv_fits(fmt, p.k_width, a.v_rank, p.vs_off, p.vq_off, p.v_nout,
                          p.v_nbo + (a.v_rank - p.v_nout + 1) / 2),
                  "decode: no P @ V window of v_rank %d fits in LDS", a.v_rank);
        if (fmt == FMT_Q4) {
            const int rk = (p.ks_off + 4 * a.Hq + 15) / 16 * 16;
            SKV_CHECK(quant_copies(rk) > 0 && quant_lds_bytes(rk, 0) <= quant_lds_limit(),
                      "decode: a 3.2-bit page of %d K bytes per row does not fit in LDS", rk);
            p.row_g = rk / 16;
            p.nch = quant_chunks(rk);
            p.lds_bytes = quant_lds_bytes(rk, 0);
        } else {
            SKV_CHECK(lowrank_copies(p.k_width, 0) > 0, "decode: a page of k_width %d does not fit in LDS",
                      p.k_width);
            p.nch = lowrank_chunks(p.k_width, 0);
            p.lds_bytes = lowrank_lds_bytes(p.k_width, 0);
        }
    } else if (fmt == FMT_Q4) {
        qnb = quant_v_blocks(a.v_rank, p.v_nout);
        p.nch = quant_chunks(row_bytes);
        p.lds_bytes = quant_lds_bytes(row_bytes, qnb);
    } else {
        p.nch = lowrank_chunks(p.k_width, nb);
        p.lds_bytes = lowrank_lds_bytes(p.k_width, nb);
    }
    p.ws = (uint8_t*)a.ws;
    p.ws_plan = wl.plan; p.ws_ab = wl.ab;
    p.ws_m = wl.m; p.ws_l = wl.l; p.ws_acc = wl.acc;
    p.ws_lg = wl.lg; p.lcap = lcap;
    p.ws_o = wl.o; p.acc_ld = wl.ld;
    p.pv_r = pv_r;
    p.ws_pages = wl.pages;

    const bool timed = g_prof.on && 2 * g_prof.used + 1 < (int)g_prof.ev.size();
    if (timed && g_prof.mode == 1) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used], stream));
    PrepArgs pa;
    pa.seq_lens = a.seq_lens; pa.n = a.n; pa.max_seq_len = a.max_seq_len; pa.grid = a.grid;
    pa.Hq = a.Hq; pa.Hkv = a.Hkv; pa.TT = TT; pa.k_rows = p.k_width;
    pa.k_ranks = a.k_ranks; pa.k_offsets = a.k_offsets;
    pa.t_head = a.t_head; pa.t_nout = a.t_nout; pa.t_last = a.t_last;
    pa.head0 = a.head0; pa.code0 = a.code0;
    pa.q = a.q; pa.q_s0 = a.q_s0; pa.q_s1 = a.q_s1; pa.q_dt = a.q_dt;
    pa.k_up = a.k_up; pa.ku_s0 = a.ku_s0; pa.ku_dt = a.w_dt;
    pa.sc = a.scale * LOG2E;
    pa.ws = p.ws; pa.ws_plan = wl.plan; pa.ws_ab = wl.ab;
    pa.tile_pairs = (TT + 1) / 2;
    pa.fold_wgs = pa.tile_pairs * ((a.n + PREP_REQ - 1) / PREP_REQ);
    pa.pages = (PageRec*)(p.ws + wl.pages);
    pa.cache = p.cache; pa.c_s0 = p.c_s0; pa.c_s1 = p.c_s1; pa.bs_shift = p.bs_shift;
    pa.bt = a.bt; pa.bt_s0 = a.bt_s0; pa.bt_s1 = a.bt_s1;
    const int64_t rec_wgs = ((int64_t)a.n * pages_of(a.max_seq_len) + PREP_RECS - 1) / PREP_RECS;
    SKV_CHECK(2 + pa.fold_wgs + rec_wgs < ((int64_t)1 << 31), "decode: %d requests x %d tokens", a.n,
              a.max_seq_len);
    const int prep_grid = 2 + pa.fold_wgs + (int)rec_wgs;
    PendingGemm pg;
    if (pending_write_on(stream, &pg)) {
        // A deferred write on this stream: its GEMM rides in prep's launch, its store
        // follows, and the decode kernels read the cache after both.
        const int64_t gw = pg.direct ? (int64_t)pg.d.jobs : (int64_t)pg.gx * pg.gy * pg.gz;
        SKV_CHECK(prep_grid + gw < ((int64_t)1 << 31), "decode: %d prep and %lld write workgroups", prep_grid,
                  (long long)gw);
        if (pg.direct) {
            const void* fn = pg.w_dtype == STARKV_BF16 ? write_prep_direct_fn<STARKV_BF16>(pg.d.n, pg.d.slices)
                                                       : write_prep_direct_fn<STARKV_F16>(pg.d.n, pg.d.slices);
            int pw = prep_grid;
            void* args[] = {(void*)&pa, (void*)&pg.d, (void*)&pw};
            SKV_HIP(hipLaunchKernel(fn, dim3(prep_grid + (int)gw), dim3(PREP_THR), args, 0, stream));
        } else if (pg.w_dtype == STARKV_BF16)
            hipLaunchKernelGGL(write_prep_kernel<STARKV_BF16>, dim3(prep_grid + (int)gw), dim3(PREP_THR), 0, stream,
                               pa, pg.g, prep_grid, pg.gx, pg.gy);
        else
            hipLaunchKernelGGL(write_prep_kernel<STARKV_F16>, dim3(prep_grid + (int)gw), dim3(PREP_THR), 0, stream,
                               pa, pg.g, prep_grid, pg.gx, pg.gy);
        SKV_HIP(hipGetLastError());
        // A direct 3.2-bit write's V latents are packed by the logits pass of a two-pass
        // decode (P @ V, a later launch, reads them), else by their own launch.
        if (!(two && fmt == FMT_Q4 && take_pending_vpack(&p.vp))) {
            const int wrc = launch_pending_store();
            if (wrc) return wrc;
        }
    } else {
        const int wrc = flush_pending_write();  // a deferred write on another stream: its own launches
        if (wrc) return wrc;
        hipLaunchKernelGGL(prep_kernel, dim3(prep_grid), dim3(PREP_THR), 0, stream, pa);
    }
    SKV_HIP(hipGetLastError());
    if (timed && g_prof.mode == 0) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used], stream));
    int rc;
    if (two) {
        rc = fmt == FMT_Q4 ? launch_quant(p, 0, a.grid, stream) : launch_lowrank(p, fmt, 0, a.grid, stream);
        if (rc) {
            if (p.vp.n > 0) launch_vpack_on(p.vp, stream);  // the logits pass did not run: the write still lands
            return rc;
        }
        SKV_HIP(hipGetLastError());
        rc = launch_pv(p, fmt, a.grid, stream);
    } else {
        rc = fmt == FMT_Q4 ? launch_quant(p, qnb, a.grid, stream) : launch_lowrank(p, fmt, nb, a.grid, stream);
    }
    if (rc) return rc;
    SKV_HIP(hipGetLastError());
    if (timed && g_prof.mode == 0) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used + 1], stream));
    if (two) {
        rc = launch_merge_wide(p, a.grid, a.vu_dt, a.vup, a.vu_s0, a.vu_s1, a.out, a.o_s0, a.o_s1, a.out_dt, stream);
    } else {
        const dim3 mgrid((a.n + MERGE_REQ - 1) / MERGE_REQ, a.Hq);
        const size_t mlds = merge_lds_bytes(a.v_rank, a.vu_dt);
        rc = a.vu_dt == STARKV_BF16  ? launch_merge<uint16_t>(mgrid, mlds, stream, p, wl, a)
             : a.vu_dt == STARKV_F16 ? launch_merge<_Float16>(mgrid, mlds, stream, p, wl, a)
                                     : launch_merge<float>(mgrid, mlds, stream, p, wl, a);
    }
    if (rc) return rc;
    SKV_HIP(hipGetLastError());
    if (timed && g_prof.mode == 1) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used + 1], stream));
    if (timed) ++g_prof.used;
    return STARKV_OK;
}

// Workspace of starkv_lowrank_decode_noalloc: one array per device, held until the
// process ends. Host code never uses the array's name as an address (on the host it
// only stands for the symbol); it uses the device address hipGetSymbolAddress returns,
// looked up once per device.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static int scratch_address(void** out) {
    static void* ptr[64] = {nullptr};
    int dev = 0;
    SKV_HIP(hipGetDevice(&dev));
    SKV_CHECK(dev >= 0 && dev < 64, "decode_noalloc: device %d", dev);
    if (!ptr[dev]) {
        void* a = nullptr;
        SKV_HIP(hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)));
        SKV_CHECK(a != nullptr && ((uintptr_t)a % 256) == 0, "decode_noalloc: scratch address");
        ptr[dev] = a;
    }
    *out = ptr[dev];
    return STARKV_OK;
}

}  // namespace starkv

using namespace starkv;

extern "C" {

int starkv_decode_grid(int n, int max_seq_len) { return grid_for(n, max_seq_len); }

int starkv_decode_grid_for(int cache_kind, int n, int num_heads, int num_kv_heads, int k_width, int v_rank,
                           int max_seq_len) {
    if (n < 1 || num_heads < 1 || num_kv_heads < 1 || k_width < 16 || v_rank < 1) return grid_for(n, max_seq_len);
    (void)cache_kind;  // the one-pass kernels and the logits pass of two-pass calls split alike
    return grid_for(n, max_seq_len, 64);
}

int starkv_profile_begin(int max_calls, int mode) {
    clear_error();
    SKV_CHECK(max_calls >= 1 && max_calls <= 100000, "profile_begin: max_calls %d", max_calls);
    SKV_CHECK(mode == 0 || mode == 1, "profile_begin: mode %d (0 decode kernels, 1 whole call)", mode);
    g_prof.mode = mode;
    for (hipEvent_t e : g_prof.ev) (void)hipEventDestroy(e);
    g_prof.ev.assign(2 * (size_t)max_calls, nullptr);
    // Timing-only events: without the system-scope fence a record does not write back
    // and invalidate the caches between the launches it separates.
    for (auto& e : g_prof.ev) SKV_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    g_prof.used = 0;
    g_prof.on = true;
    return STARKV_OK;
}

int starkv_profile_end(double* decode_ms_sum, int* calls) {
    clear_error();
    g_prof.on = false;
    double sum = 0.0;
    g_prof.ms.assign(g_prof.used, 0.0);
    for (int i = 0; i < g_prof.used; ++i) {
        SKV_HIP(hipEventSynchronize(g_prof.ev[2 * i + 1]));
        float ms = 0.f;
        SKV_HIP(hipEventElapsedTime(&ms, g_prof.ev[2 * i], g_prof.ev[2 * i + 1]));
        g_prof.ms[i] = ms;
        sum += ms;
    }
    if (decode_ms_sum) *decode_ms_sum = sum;
    if (calls) *calls = g_prof.used;
    g_prof.used = 0;
    return STARKV_OK;
}

int starkv_profile_times(double* ms, int max) {
    clear_error();
    SKV_CHECK(ms != nullptr && max >= 0, "profile_times: null output");
    const int k = std::min(max, (int)g_prof.ms.size());
    for (int i = 0; i < k; ++i) ms[i] = g_prof.ms[i];
    return k;
}

size_t starkv_decode_workspace_bytes(int cache_kind, int n, int num_heads, int num_kv_heads, int k_width, int v_rank,
                                     int max_seq_len, int grid) {
    if (n < 1 || num_heads < 1 || num_kv_heads < 1 || k_width < 16 || v_rank < 1 || max_seq_len < 1 || grid < 1)
        return 0;
    int fmt, row_bytes, v_nout = 0, TT;
    if (cache_kind == STARKV_CACHE_Q3_2) {
        if (k_width % 16) return 0;
        return starkv_quant_group_workspace_bytes(n, k_width, num_heads, v_rank, 0, num_heads, 0, k_width,
                                                  max_seq_len, grid);
    } else {
        fmt = cache_kind == STARKV_F16 ? FMT_F16 : FMT_BF16;
        row_bytes = (k_width + v_rank) * 2;
        TT = (num_heads / num_kv_heads) * (k_width / 16);
    }
    const bool two = use_two_pass(fmt, k_width, v_rank, row_bytes, v_nout, TT);
    return ws_layout(n, num_heads, TT, v_rank, grid, two ? lcap_of(max_seq_len) : 0,
                     two ? pv_ratio(fmt, n, max_seq_len, grid) : 1, pages_of(max_seq_len))
        .total;
}

int starkv_decode_layer_fits(int cache_kind, int num_heads, int num_kv_heads, const int32_t* k_ranks, int v_rank) {
    clear_error();
    SKV_CHECK(k_ranks != nullptr, "decode_layer_fits: null k_ranks");
    SKV_CHECK(num_heads >= 1 && num_kv_heads >= 1 && num_heads % num_kv_heads == 0,
              "decode_layer_fits: %d query heads over %d kv heads", num_heads, num_kv_heads);
    if (cache_kind == STARKV_CACHE_Q3_2)
        return num_heads == num_kv_heads && quant_group_fits(k_ranks, num_heads, v_rank, 0, num_heads);
    return codes_group_fits(cache_kind, num_heads / num_kv_heads, k_ranks, num_kv_heads, v_rank);
}

int starkv_decode_layer_groups(int cache_kind, int num_heads, int num_kv_heads, const int32_t* k_ranks, int v_rank,
                               int32_t* groups, int max_groups) {
    clear_error();
    if (k_ranks == nullptr || groups == nullptr || max_groups < 1 || num_heads < 1 || num_kv_heads < 1 ||
        num_heads % num_kv_heads != 0) {
        set_error("decode_layer_groups: %d query heads over %d kv heads, %d group slots", num_heads, num_kv_heads,
                  max_groups);
        return -1;
    }
    const bool quant = cache_kind == STARKV_CACHE_Q3_2;
    if (quant && num_heads != num_kv_heads) return 0;  // MHA only (paged_quant.py:374)
    const int per = num_heads / num_kv_heads;
    auto fits = [&](int g0, int g1) {
        return quant ? quant_group_fits(k_ranks, num_kv_heads, v_rank, g0, g1)
                     : codes_group_fits(cache_kind, per, k_ranks + g0, g1 - g0, v_rank);
    };
    int count = 0;
    for (int g0 = 0; g0 < num_kv_heads;) {
        if (!fits(g0, g0 + 1)) return 0;
        int g1 = g0 + 1;
        while (g1 < num_kv_heads && fits(g0, g1 + 1)) ++g1;
        if (count == max_groups) return 0;
        groups[2 * count] = g0;
        groups[2 * count + 1] = g1;
        ++count;
        g0 = g1;
    }
    return count;
}

int starkv_decode_set_path(int mode) {
    clear_error();
    if (mode < 0 || mode > 2) {
        set_error("decode_set_path: mode %d (0 auto, 1 one-pass, 2 two-pass)", mode);
        return -1;
    }
    const int prev = g_path;
    g_path = mode;
    return prev;
}

int starkv_decode_two_pass(int cache_kind, int num_heads, int num_kv_heads, int k_width, int v_rank) {
    if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0 || k_width < 16) return 0;
    if (cache_kind == STARKV_CACHE_Q3_2)
        return starkv_quant_group_two_pass(k_width, num_heads, v_rank, 0, num_heads, 0, k_width);
    return use_two_pass(cache_kind == STARKV_F16 ? FMT_F16 : FMT_BF16, k_width, v_rank, (k_width + v_rank) * 2, 0,
                        num_heads / num_kv_heads * (k_width / 16));
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
                          int v_col, const void* v_up_by_q, int64_t vu_s0, int64_t vu_s1, int vu_dtype, int v_rank,
                          const void* cos_sin, int64_t cs_s0, int cs_dtype, float scale, void* out, int64_t o_s0,
                          int64_t o_s1, int out_dtype, void* workspace, size_t workspace_bytes, int grid) {
    clear_error();
    SKV_CHECK(code_dtype == STARKV_BF16 || code_dtype == STARKV_F16, "lowrank_decode: codes must be bf16 or fp16");
    SKV_CHECK(num_kv_heads >= 1 && num_heads % num_kv_heads == 0, "lowrank_decode: num_heads %% num_kv_heads != 0");
    SKV_CHECK(k_width >= 16 && k_width % 16 == 0, "lowrank_decode: k_width %d must be a positive multiple of 16",
              k_width);
    SKV_CHECK(v_col >= k_width && v_col % 8 == 0, "lowrank_decode: v_col %d must be >= k_width %d and a multiple of 8",
              v_col, k_width);
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
    p.v_col = v_col;
    CommonArgs a{query, q_s0, q_s1, q_dtype, block_table, bt_s0, bt_s1, seq_lens, n, num_heads, num_kv_heads,
                 max_seq_len, k_up, ku_s0, w_dtype, k_ranks, k_head_offsets, nullptr, nullptr, nullptr, 0, 0,
                 v_up_by_q, vu_s0, vu_s1, vu_dtype, v_rank, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1,
                 out_dtype, workspace, workspace_bytes, grid};
    const int TT = (num_heads / num_kv_heads) * (k_width / 16);
    // A row holds, from the cache pointer, the K lanes read and then the V codes at v_col.
    return decode_common(p, a, code_dtype == STARKV_BF16 ? FMT_BF16 : FMT_F16, (v_col + v_rank) * 2, TT,
                         (hipStream_t)stream);
}

int starkv_lowrank_decode_noalloc(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                                  const void* kv_cache, int64_t c_s0, int64_t c_s1, int code_dtype, int block_size,
                                  const int32_t* block_table, int64_t bt_s0, int64_t bt_s1, const int32_t* seq_lens,
                                  int n, int num_heads, int num_kv_heads, int max_seq_len, const void* k_up,
                                  int64_t ku_s0, int w_dtype, const int32_t* k_ranks, const int32_t* k_head_offsets,
                                  int k_width, int v_col, const void* v_up_by_q, int64_t vu_s0, int64_t vu_s1,
                                  int vu_dtype,
                                  int v_rank, const void* cos_sin, int64_t cs_s0, int cs_dtype, float scale,
                                  void* out, int64_t o_s0, int64_t o_s1, int out_dtype, int grid) {
    clear_error();
    SKV_CHECK(code_dtype == STARKV_BF16 || code_dtype == STARKV_F16,
              "lowrank_decode_noalloc: codes must be bf16 or fp16");
    const size_t need = starkv_decode_workspace_bytes(code_dtype, n, num_heads, num_kv_heads, k_width, v_rank,
                                                      max_seq_len, grid);
    SKV_CHECK(need > 0, "lowrank_decode_noalloc: invalid sizes");
    SKV_CHECK(need <= NOALLOC_SCRATCH_BYTES,
              "lowrank_decode_noalloc: this call needs %zu workspace bytes, more than the %zu of the "
              "library's fixed scratch (use starkv_lowrank_decode with a workspace, or fewer requests)",
              need, NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc) return rc;
    return starkv_lowrank_decode(stream, query, q_s0, q_s1, q_dtype, kv_cache, c_s0, c_s1, code_dtype, block_size,
                                 block_table, bt_s0, bt_s1, seq_lens, n, num_heads, num_kv_heads, max_seq_len, k_up,
                                 ku_s0, w_dtype, k_ranks, k_head_offsets, k_width, v_col, v_up_by_q, vu_s0, vu_s1,
                                 vu_dtype, v_rank, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1, out_dtype, ws,
                                 NOALLOC_SCRATCH_BYTES, grid);
}

int starkv_quant_decode_group(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                              const uint8_t* kv_cache, int64_t c_s0, int64_t c_s1, int block_size,
                              const int32_t* block_table, int64_t bt_s0, int64_t bt_s1, const int32_t* seq_lens, int n,
                              int num_heads, int max_seq_len, int k_width, int v_rank, int row_bytes,
                              const void* k_up, int64_t ku_s0, int w_dtype, const int32_t* tile_head,
                              const int32_t* tile_nout, const int32_t* tile_last, const void* v_up_by_q,
                              int64_t vu_s0, int64_t vu_s1, int vu_dtype, const void* cos_sin, int64_t cs_s0,
                              int cs_dtype, float scale, void* out, int64_t o_s0, int64_t o_s1, int out_dtype,
                              void* workspace, size_t workspace_bytes, int grid, int row_k_width, int row_num_heads,
                              int head0, int k_lane0) {
    clear_error();
    SKV_CHECK(qgroup_args_ok(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0, k_width),
              "quant_decode: heads [%d, %d) with K lanes [%d, %d) of a layer of %d heads and K width %d "
              "(widths multiples of 16)",
              head0, head0 + num_heads, k_lane0, k_lane0 + k_width, row_num_heads, row_k_width);
    SKV_CHECK(query && kv_cache && block_table && seq_lens && k_up && tile_head && tile_nout && tile_last &&
                  v_up_by_q && cos_sin && out && workspace,
              "quant_decode: null pointer");
    const QGroup g = qgroup(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0);
    SKV_CHECK(row_bytes == g.row.nbytes, "quant_decode: row_bytes %d != QuantRow.nbytes %d", row_bytes,
              g.row.nbytes);
    DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.cache = kv_cache + g.base;
    p.c_s0 = c_s0;
    p.c_s1 = c_s1;
    p.bs_shift = block_shift(block_size);
    p.k_width = k_width;
    p.v_nout = g.row.v_nout;
    p.v_nbo = g.row.v_nbo;
    p.ks_off = g.ks_off;
    p.vs_off = g.vs_off;
    p.vq_off = g.vq_off;
    CommonArgs a{query, q_s0, q_s1, q_dtype, block_table, bt_s0, bt_s1, seq_lens, n, num_heads, num_heads,
                 max_seq_len, k_up, ku_s0, w_dtype, nullptr, nullptr, tile_head, tile_nout, tile_last, head0, g.code0,
                 v_up_by_q, vu_s0, vu_s1, vu_dtype, v_rank, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1,
                 out_dtype, workspace, workspace_bytes, grid};
    return decode_common(p, a, FMT_Q4, g.extent, k_width / 16, (hipStream_t)stream);
}

int starkv_quant_decode(void* stream, const void* query, int64_t q_s0, int64_t q_s1, int q_dtype,
                        const uint8_t* kv_cache, int64_t c_s0, int64_t c_s1, int block_size,
                        const int32_t* block_table, int64_t bt_s0, int64_t bt_s1, const int32_t* seq_lens, int n,
                        int num_heads, int max_seq_len, int k_width, int v_rank, int row_bytes, const void* k_up,
                        int64_t ku_s0, int w_dtype, const int32_t* tile_head, const int32_t* tile_nout,
                        const int32_t* tile_last, const void* v_up_by_q, int64_t vu_s0, int64_t vu_s1,
                        int vu_dtype, const void* cos_sin, int64_t cs_s0, int cs_dtype, float scale, void* out,
                        int64_t o_s0, int64_t o_s1, int out_dtype, void* workspace, size_t workspace_bytes,
                        int grid) {
    return starkv_quant_decode_group(stream, query, q_s0, q_s1, q_dtype, kv_cache, c_s0, c_s1, block_size,
                                     block_table, bt_s0, bt_s1, seq_lens, n, num_heads, max_seq_len, k_width, v_rank,
                                     row_bytes, k_up, ku_s0, w_dtype, tile_head, tile_nout, tile_last, v_up_by_q,
                                     vu_s0, vu_s1, vu_dtype, cos_sin, cs_s0, cs_dtype, scale, out, o_s0, o_s1,
                                     out_dtype, workspace, workspace_bytes, grid, k_width, num_heads, 0, 0);
}

size_t starkv_quant_group_workspace_bytes(int n, int row_k_width, int row_num_heads, int v_rank, int head0,
                                          int num_heads, int k_lane0, int k_width, int max_seq_len, int grid) {
    if (n < 1 || max_seq_len < 1 || grid < 1 ||
        !qgroup_args_ok(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0, k_width))
        return 0;
    const QGroup g = qgroup(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0);
    const bool two = qgroup_two_pass(g, k_width);
    return ws_layout(n, num_heads, k_width / 16, v_rank, grid, two ? lcap_of(max_seq_len) : 0,
                     two ? pv_ratio(FMT_Q4, n, max_seq_len, grid) : 1, pages_of(max_seq_len))
        .total;
}

int starkv_quant_group_two_pass(int row_k_width, int row_num_heads, int v_rank, int head0, int num_heads,
                                int k_lane0, int k_width) {
    if (!qgroup_args_ok(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0, k_width)) return 0;
    return qgroup_two_pass(qgroup(row_k_width, row_num_heads, v_rank, head0, num_heads, k_lane0), k_width);
}

}  // extern "C"
