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
//    per-wave accumulators.
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
                                                     const int32_t* __restrict__ t_last, uint8_t* __restrict__ ws,
                                                     size_t ws_tiles, size_t ws_plan) {
    __shared__ int s_wsum[16];
    __shared__ int s_total;
    __shared__ int s_hf[MAX_H], s_hn[MAX_H];
    __shared__ int s_rank[MAX_H], s_off[MAX_H];        // k_ranks, k_offsets (bf16/fp16)
    __shared__ int s_thead[MAX_TT], s_tmeta[MAX_TT];   // t_head, nout | last << 8 (3.2-bit)
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
        for (int t = tid; t < TT; t += blockDim.x)
            tiles[t] = make_int4(s_thead[t], 16 * t, 16 | ((s_tmeta[t] & 255) << 8) | ((s_tmeta[t] >> 8) << 16),
                                 s_thead[t]);
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
        for (int j = 0; j < nt && t0 + j < TT; ++j, ++cnt)
            tiles[t0 + j] = make_int4(tid, o + 16 * j, min(16, R - 16 * j) | ((j == nt - 1) << 16), kv);
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
        // order, sl = their tiles. Lane w < 8 also counts its wave's heads and tiles.
        int k = 0, sl = 0, nhw = 0, ntw = 0;
        for (int h = 0; h < Hq; ++h) {
            const int wh = __builtin_amdgcn_readlane(hwave, h), ph = __builtin_amdgcn_readlane(pos, h);
            const int zh = __builtin_amdgcn_readlane(hsz, h);
            if (wh == hwave && ph < pos) { ++k; sl += zh; }
            if (wh == lane) { ++nhw; ntw += zh; }
        }
        // Clear the 8 plans, then every head writes its own entries (same wave: in order).
        for (int i = lane; i < NWAVE * PLAN_STRIDE; i += 64) plan[i] = 0;
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): the clears land first
        if (lane < Hq && ok) {
            int* pw = plan + hwave * PLAN_STRIDE;
            pw[32 + k] = lane;
            pw[40 + k] = sl;
            pw[48 + k] = hsz;
            for (int j = 0; j < hsz; ++j) pw[8 + sl + j] = hfirst + j;
        }
        if (lane < NWAVE) {
            int* pw = plan + lane * PLAN_STRIDE;
            pw[0] = ok ? ntw : 0;
            pw[1] = ok ? nhw : 0;
        }
        if (lane == 0) plan[NWAVE * PLAN_STRIDE] = ok;
    }
}

// ---------------------------------------------------------------------------
// 2. fold: AB[b][t][ks][lane] = 8 fp16 of tile row m = lane & 15, columns
//    32 ks + 8 (lane >> 4) .. +8, scaled by scale*log2(e); rows past the head's rank
//    are zero (paged_decode.py:79-81 masks them). Row m holds rank m of the tile, or,
//    for the 3.2-bit cache (perm = 1), rank (m >> 2) + 4 (m & 3): then the z values a
//    lane receives (rows 4g .. 4g+3) are ranks g, g+4, g+8, g+12, whose codes are the
//    nibbles a lane extracts from the tile's 8 bytes with one shift.
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
    const int rr = perm ? (m >> 2) + 4 * (m & 3) : m;
    const int c0 = 32 * k2 + 8 * lg;
    const int64_t ur = (int64_t)(tm.y + rr) * ku_s0;
    const int64_t qh = (int64_t)b * q_s0 + (int64_t)tm.x * q_s1;
    const float s = rr < (tm.z & 255) ? sc : 0.f;
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
// 3.2-bit page copies. LDS layout of a page buffer: the page's 16 cos/sin
// rows first (256 bytes each, granule c of row r stored at granule c ^ r, so the MFMA
// operand reads of 16 rows hit distinct banks: 4 copies of 1 KB), then the 16 token
// rows at a pitch of pitch_g granules (odd, so rows fall on different banks; granules
// past row_g are filler). Copy i of wave w is 1 KB chunk ch = 8 i + w; lane q of it
// moves granule 64 ch + q, whose offset inside the page's cos/sin rows or rows is the
// same for every page: `doff`. The two buffer descriptors of a page cover only the
// request's rows, so rows past its end are not read. Every wave issues exactly NLD
// copies; lanes with nothing to move (filler granules, chunks past the page, which land
// in the buffer's unused tail) carry an offset past the descriptor's range, so they
// touch no memory, and one vmcnt value covers a page on every wave.
// ---------------------------------------------------------------------------
template <int NLD>
__device__ __forceinline__ void dma_page(const DecodeParams& p, const Cursor& c, cint_p P, uint8_t* buf, int wave,
                                         const uint32_t (&doff)[MAX_NLD]) {
    // Past the end of the workgroup's range the copies still issue (with empty
    // descriptors: no memory access), so every page of the loop issues the same NLD
    // copies and the waits stay static.
    const bool v = c.valid;
    const int k = v ? c.k : 0;
    const int blk = v ? ((cint_p)p.bt)[c.b * p.bt_s0 + (k >> p.bs_shift) * p.bt_s1] : 0;
    const int row0 = (k & ((1 << p.bs_shift) - 1)) * TILE_TOK;  // first slot of the page inside its block
    const uint8_t* page = p.cache + (int64_t)blk * p.c_s0 + (int64_t)row0 * p.c_s1;
    const int tok0 = TILE_TOK * k;
    const int rows = v ? min(TILE_TOK, c.len - tok0) : 0;
    const int4v_t rkv = buffer_rsrc(page, rows * (int)p.c_s1);
    const int4v_t rcs = buffer_rsrc(p.cs + (int64_t)tok0 * p.cs_s0b, rows * p.cs_s0b);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)buf;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        const uint32_t dst = lds0 + (uint32_t)ch * 1024u;
        if (i == 0 && ch < CS_CHUNKS)
            lds_copy16(rcs, dst, doff[i]);
        else  // rows; filler granules and surplus copies carry an out-of-range offset
            lds_copy16(rkv, dst, doff[i]);
    }
}

// A lane's share of one rank tile's logit for token (lane & 15): its 4 z values (rows
// 4g .. 4g+3, g = lane >> 4) times their codes, read at byte `xoff` of the token's row.
// 3.2-bit: the codes are nibbles n with value n - 8, built as fp16 (1024 + n) - 1032
// (exact); the scales come per (token, head) from the row's bf16 (outlier, inlier) pair
// at byte `soff`, the outlier part from the lane's first k elements (k = outlier ranks
// among its 4, from the tile's count c).
template <int FMT>
__device__ __forceinline__ float tile_dot(const f32x4_t& z, const uint8_t* xr, int xoff, int soff, int c, int k,
                                          int lg, const uint2* s_kmask) {
    // One 64-bit LDS load (not two 32-bit ones the backend would pair up: the paired
    // instruction loses the memory operand that tells it apart from copies in flight).
    if (FMT == FMT_BF16) {
        const uint2 w = ld64(xr + xoff + 8 * lg);
        float v = __uint_as_float(w.x << 16) * z[0];
        v = fmaf(__uint_as_float(w.x & 0xffff0000u), z[1], v);
        v = fmaf(__uint_as_float(w.y << 16), z[2], v);
        return fmaf(__uint_as_float(w.y & 0xffff0000u), z[3], v);
    } else if (FMT == FMT_F16) {
        const uint2 w = ld64(xr + xoff + 8 * lg);
        return dot2(as_h2(w.x), cvt_h2(z[0], z[1]), dot2(as_h2(w.y), cvt_h2(z[2], z[3]), 0.f));
    } else {
        const uint2 w = ld64(xr + xoff);
        const uint32_t sh = 4 * lg;
        const half2_t off = {(_Float16)1032.f, (_Float16)1032.f};
        const half2_t x0 = as_h2(((w.x >> sh) & 0x000F000Fu) | 0x64006400u) - off;  // ranks g, g+4
        const half2_t x1 = as_h2(((w.y >> sh) & 0x000F000Fu) | 0x64006400u) - off;  // ranks g+8, g+12
        const half2_t z01 = cvt_h2(z[0], z[1]), z23 = cvt_h2(z[2], z[3]);
        const float d = dot2(x0, z01, dot2(x1, z23, 0.f));
        const uint32_t sw = *(const uint32_t*)(xr + soff);
        const float si = __uint_as_float(sw & 0xffff0000u);
        if (c == 0) return si * d;
        const uint2 mk = s_kmask[k];
        const float dout =
            dot2(as_h2(h2_bits(x0) & mk.x), z01, dot2(as_h2(h2_bits(x1) & mk.y), z23, 0.f));
        return fmaf(__uint_as_float(sw << 16), dout, si * (d - dout));
    }
}

template <int MTV>
struct WaveTiles {
    int ntw, nh;                   // rank tiles (slots) and query heads of this wave
    int xoff[MTV], meta[MTV];      // per slot: code byte offset in a row; 3.2-bit: scale offset << 8 | outliers
};

// K side of one page: MTV slots of this wave, partial logits into sp[slot][token]
// (this wave's own LDS region). Every slot is computed (slots past the wave's tiles
// use tile 0 and land in a spare row), so the compiler can hoist the LDS reads and
// interleave the MFMA chains of neighbouring slots.
template <int FMT, int MTV>
__device__ __forceinline__ void k_side(const DecodeParams& p, const WaveTiles<MTV>& wt, const half8_t (&ab)[MTV][4],
                                       const uint8_t* XC, float* sp, const uint2* s_kmask, uint32_t kpack, int lane,
                                       int wave, int cur_b) {
    const int ln = opaque(lane);  // LDS addresses are recomputed per page, not held per buffer and slot
    const int lr = ln & 15, lg = ln >> 4;
    half8_t csb[4];  // B operand: position lr of the page, K elements 32 ks + 8 lg .. +8 (granule 4 ks + lg)
    {
        const uint8_t* csr = XC + lr * CS_ROW_LDS;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) csb[ks] = *(const half8_t*)(csr + (((4 * ks + lg) ^ lr) << 4));
    }
    const uint8_t* xr = XC + CS_CHUNKS * 1024 + lr * p.pitch_b;
    const int rslot = ((lg & 1) << 1) | (lg >> 1);  // sum_rows4 puts inputs (a, b, c, d) in rows (0, 2, 1, 3)
    const int ntw = opaque_s(wt.ntw);
    float v[4];
#pragma unroll
    for (int i = 0; i < MTV; ++i) {
        const f32x4_t z = mfma_tile(ab[i], csb);
        const int meta = FMT == FMT_Q4 ? wt.meta[i] : 0;
        v[i & 3] = tile_dot<FMT>(z, xr, wt.xoff[i], meta >> 8, meta & 255, (kpack >> (3 * i)) & 7, lg, s_kmask);
        if ((i & 3) == 3 || i == MTV - 1) {  // four tiles (or the last ones): one reduction over the row groups
            const float r = sum_rows4(v[0], (i & 3) >= 1 ? v[1] : 0.f, (i & 3) >= 2 ? v[2] : 0.f,
                                      (i & 3) >= 3 ? v[3] : 0.f);
            const int slot = 4 * (i >> 2) + rslot;
            sp[(slot < ntw ? slot : MAX_SLOTS) * TILE_TOK + lr] = r;
        }
    }
    // Slots past MTV: AB from the workspace (L2) on every page.
    if (ntw > MTV) {
        cint_p plan = (cint_p)(p.ws + p.ws_plan) + wave * PLAN_STRIDE;
        cint_p tiles = (cint_p)(p.ws + p.ws_tiles);
        const half8_t* abg = (const half8_t*)(p.ws + p.ws_ab + (size_t)cur_b * p.TT * AB_TILE_BYTES);
        for (int i = MTV; i < ntw; ++i) {
            const int t = plan[8 + i];
            half8_t a[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) a[ks] = abg[(t * 4 + ks) * 64 + lane];
            const int4 tm = load_tile(tiles, t);
            const int c = (tm.z >> 8) & 255;
            const int k = min(max((c - lg + 3) >> 2, 0), 4);
            const int xoff = FMT == FMT_Q4 ? (tm.y >> 1) : 2 * tm.y;
            const float r = sum_rows(tile_dot<FMT>(mfma_tile(a, csb), xr, xoff, p.ks_off + 4 * tm.x, c, k, lg, s_kmask));
            if (lane < 16) sp[i * TILE_TOK + lr] = r;
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): no tracked load left pending
    }
}

// Returns true when some head's reference max moved (acc needs rescaling by alpha).
template <int FMT>
__device__ __forceinline__ bool softmax_page(SmState& sm, int nh, const float* sp, uint16_t* spp, uint16_t* spl,
                                             float* salpha, int lane, int tok0, int lo, int hi) {
    const int ln = opaque(lane);
    const int kh = ln >> 4, lr = ln & 15;
    float s = 0.f;
    for (int t = 0; t < sm.hn; ++t) s += sp[(sm.hf + t) * TILE_TOK + lr];
    s = tok0 + lr >= lo && tok0 + lr < hi && kh < nh ? s : -INFINITY;
    float alpha = 1.f;
    bool moved = false;
    if (__builtin_amdgcn_ballot_w64(s > sm.m + LAZY_MAX) != 0) {
        const float mn = fmaxf(sm.m, row16_max(s));
        alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(sm.m - mn);
        sm.m = mn;
        moved = true;
    }
    const float pe = s == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - sm.m);
    sm.l = fmaf(sm.l, alpha, pe);
    const int idx = kh * TILE_TOK + lr;  // rows past the wave's heads hold P = 0
    if (FMT == FMT_BF16) {
        // P = hi + lo in two bfloat16 parts: the P @ V product keeps ~16 bits of P.
        const __bf16 ph = (__bf16)pe;
        const __bf16 pl = (__bf16)(pe - (float)ph);
        spp[idx] = __builtin_bit_cast(uint16_t, ph);
        spl[idx] = __builtin_bit_cast(uint16_t, pl);
    } else {
        spp[idx] = __builtin_bit_cast(uint16_t, (_Float16)pe);
    }
    if (lr == 0) salpha[kh] = alpha;
    return moved;
}

// acc[nb] = alpha * acc[nb] + P[4 heads, 16 tokens] @ V[16 tokens, 64 columns] for page
// X, on v_mfma_f32_4x4x4_16b with block 0's A broadcast (cbsz 4): per 4-token step,
// lanes 0..3 hold P[head l][4 tokens], lane l holds V[4 tokens][column 64 nb + l], and
// the result lands in lane l as acc[nb][head] for its column.
template <int FMT, int NB>
__device__ __forceinline__ void pv_page(const DecodeParams& p, f32x4_t (&acc)[NB], const uint8_t* X,
                                        const uint16_t* spp, const uint16_t* spl, const float* salpha, bool rescale,
                                        int lane) {
    const int ln = opaque(lane);
    if (rescale) {
        const f32x4_t al = *(const f32x4_t*)salpha;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[nb][e] *= al[e];
    }
    const uint8_t* rows = X + CS_CHUNKS * 1024;
    const uint16_t* pr = spp + (ln & 3) * TILE_TOK;
    const uint16_t* plr = spl + (ln & 3) * TILE_TOK;
#pragma unroll
    for (int st = 0; st < 4; ++st) {  // tokens 4 st .. 4 st + 3
        const uint2 pa = *(const uint2*)(pr + 4 * st);
        const uint2 pl = FMT == FMT_BF16 ? *(const uint2*)(plr + 4 * st) : make_uint2(0, 0);
        const uint8_t* r0 = rows + 4 * st * p.pitch_b;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int c = 64 * nb + ln;  // columns past v_rank compute garbage that is never stored
            uint32_t b0, b1;
            if (FMT == FMT_Q4) {
                const bool o = c < p.v_nout;
                const int ci = o ? c : c - p.v_nout;
                const int vb = p.vq_off + (o ? 0 : p.v_nbo) + (ci >> 1);
                const int vsh = 4 * (ci & 1);
                const int vso = p.vs_off + (o ? 0 : 2);
                float val[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint8_t* rp = r0 + e * p.pitch_b;
                    const int nib = (int)((rp[vb] >> vsh) & 15u) - 8;
                    val[e] = (float)nib * __uint_as_float((uint32_t)(*(const uint16_t*)(rp + vso)) << 16);
                }
                b0 = h2_bits(cvt_h2(val[0], val[1]));
                b1 = h2_bits(cvt_h2(val[2], val[3]));
            } else {
                const uint8_t* vp = r0 + 2 * (p.k_width + c);
                const uint32_t u0 = *(const uint16_t*)vp, u1 = *(const uint16_t*)(vp + p.pitch_b);
                const uint32_t u2 = *(const uint16_t*)(vp + 2 * p.pitch_b), u3 = *(const uint16_t*)(vp + 3 * p.pitch_b);
                b0 = u0 | (u1 << 16);
                b1 = u2 | (u3 << 16);
            }
            const uint2 bv = make_uint2(b0, b1);
            if (FMT == FMT_BF16) {
                acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(short4_t, pa),
                                                                 __builtin_bit_cast(short4_t, bv), acc[nb], 4, 0, 0);
                acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(short4_t, pl),
                                                                 __builtin_bit_cast(short4_t, bv), acc[nb], 4, 0, 0);
            } else {
                acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, pa),
                                                             __builtin_bit_cast(half4_t, bv), acc[nb], 4, 0, 0);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// One page of the decode loop: XC holds page j (copied two pages ago) and XN receives
// page j + 2 (its previous page, j - 1, is finished on every wave once the barrier is
// passed). Distinct __shared__ arrays per buffer keep every address static.
// ---------------------------------------------------------------------------
template <int FMT, int MTV, int NB, int NLD>
__device__ __forceinline__ bool decode_iter(LoopState& st, const WaveTiles<MTV>& wt, half8_t (&ab)[MTV][4],
                                            f32x4_t (&acc)[NB], SmState& sm, const uint32_t (&doff)[MAX_NLD],
                                            uint32_t kpack, const uint8_t* XC, uint8_t* XN, float* sp,
                                            uint16_t* spp, uint16_t* spl, float* salpha, const uint2* s_kmask,
                                            const int* sqh, int lane, int wave) {
    const DecodeParams& p = params();
    cint_p P = (cint_p)(p.ws + 4);
    if (!st.cc.valid) return false;
    const Cursor cc = st.cc;
    if (st.new_seg) {
        // This request's AB into registers; slots past the wave's tiles load tile 0.
        cint_p plan = (cint_p)(p.ws + p.ws_plan) + wave * PLAN_STRIDE;
        const half8_t* abp = (const half8_t*)(p.ws + p.ws_ab + (size_t)cc.b * p.TT * AB_TILE_BYTES);
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            const int t = plan[8 + i];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ab[i][ks] = abp[(t * 4 + ks) * 64 + lane];
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    }
    SKV_WAIT_VM_LGKM0(NLD);  // only the copies of page j + 1 may still be in flight
    lds_barrier();           // page j is in LDS; every wave is done with page j - 1
    dma_page<NLD>(p, st.ld, P, XN, opaque_s(wave), doff);
    if (st.ld.valid) cur_next(st.ld, P, p.n, st.beg, st.end);
    k_side<FMT, MTV>(p, wt, ab, XC, sp, s_kmask, kpack, lane, wave, cc.b);
    const bool moved = softmax_page<FMT>(sm, wt.nh, sp, spp, spl, salpha, lane, TILE_TOK * cc.k, cc.lo, cc.hi);
    pv_page<FMT, NB>(p, acc, XC, spp, spl, salpha, moved, lane);
    Cursor nx = cc;
    const bool seg_end = cur_next(nx, P, p.n, st.beg, st.end);
    if (seg_end) flush_partial<NB>(p, sm, acc, wt.nh, cc.b + st.g, sqh, lane);
    st.cc = nx;
    st.new_seg = seg_end;
    ++st.j;
    return true;
}

// ---------------------------------------------------------------------------
// 3. decode. MTV = rank tiles per wave held in VGPRs (more stream from L2); NB =
//    64-column blocks of V; XB = bytes per page buffer; NLD = copies per lane per page.
// ---------------------------------------------------------------------------
template <int FMT, int MTV, int NB, int XB, int NLD>
__global__ __launch_bounds__(NTHR) void decode_kernel(const DecodeParams p0) {
    __shared__ __attribute__((aligned(16))) uint8_t s_x0[XB];
    __shared__ __attribute__((aligned(16))) uint8_t s_x1[XB];
    __shared__ __attribute__((aligned(16))) uint8_t s_x2[XB];
    __shared__ __attribute__((aligned(16))) float s_part[NWAVE][(MAX_SLOTS + 1) * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_p[NWAVE][4 * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_plo[FMT == FMT_BF16 ? NWAVE : 1][4 * TILE_TOK];
    __shared__ __attribute__((aligned(16))) float s_alpha[NWAVE][4];
    __shared__ __attribute__((aligned(16))) uint2 s_kmask[8];
    __shared__ int s_qh[NWAVE][4];

    const DecodeParams& p = params();
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    const int lg = lane >> 4;
    cint_p P = (cint_p)(p.ws + 4);
    cint_p plan = (cint_p)(p.ws + p.ws_plan);
    if (plan[NWAVE * PLAN_STRIDE] == 0) return;  // no wave plan: the merge reports NaN
    LoopState st;
    st.g = blockIdx.x;
    const int S_tok = ((cint_p)p.ws)[0];
    const int T = P[p.n];
    st.beg = min(st.g * S_tok, T);
    st.end = min(st.beg + S_tok, T);
    if (st.beg >= st.end) return;

    // Page buffers start zeroed: rows past a request's end are never copied, and
    // must hold finite values (P is 0 there).
    for (int i = tid; i < XB / 16; i += NTHR) {
        ((uint4*)s_x0)[i] = make_uint4(0, 0, 0, 0);
        ((uint4*)s_x1)[i] = make_uint4(0, 0, 0, 0);
        ((uint4*)s_x2)[i] = make_uint4(0, 0, 0, 0);
    }
    if (tid < NWAVE * 4) (&s_alpha[0][0])[tid] = 1.f;
    if (tid < 8) {  // fp16-pair masks of a lane's first k elements (pairs (0,1), (2,3))
        const uint32_t m0 = tid >= 2 ? 0xffffffffu : tid == 1 ? 0x0000ffffu : 0u;
        const uint32_t m1 = tid >= 4 ? 0xffffffffu : tid == 3 ? 0x0000ffffu : 0u;
        s_kmask[tid] = make_uint2(m0, m1);
    }

    // This wave's plan: slots (rank tiles) and heads (at most 4: Hq <= 32).
    cint_p pw = plan + wave * PLAN_STRIDE;
    WaveTiles<MTV> wt;
    wt.ntw = pw[0];
    wt.nh = pw[1];
    uint32_t kpack = 0;
    {
        cint_p tiles = (cint_p)(p.ws + p.ws_tiles);
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            const int4 tm = load_tile(tiles, pw[8 + i]);
            wt.xoff[i] = FMT == FMT_Q4 ? (tm.y >> 1) : 2 * tm.y;
            const int c = (tm.z >> 8) & 255;
            wt.meta[i] = ((p.ks_off + 4 * tm.x) << 8) | c;
            if (FMT == FMT_Q4) kpack |= (uint32_t)min(max((c - lg + 3) >> 2, 0), 4) << (3 * i);
        }
    }
    if (lane < 4) s_qh[wave][lane] = lane < wt.nh ? ((const int*)pw)[32 + lane] : 0;
    SmState sm;
    sm.hf = lg < wt.nh ? ((const int*)pw)[40 + lg] : 0;
    sm.hn = lg < wt.nh ? ((const int*)pw)[48 + lg] : 0;
    sm.m = -INFINITY;
    sm.l = 0.f;
    // Copy offsets of this lane inside a page (chunks 0..3: cos/sin rows; then rows).
    uint32_t doff[MAX_NLD];
#pragma unroll
    for (int i = 0; i < MAX_NLD; ++i) {
        const int ch = i * NWAVE + wave;
        uint32_t off = 0x80000000u;  // past the descriptor range: no memory access
        if (i < NLD) {
            if (ch < CS_CHUNKS) {
                const int g = ch * 64 + lane, row = g >> 4;  // LDS granule g holds granule (g & 15) ^ row
                off = (uint32_t)(row * p.cs_s0b + (((g & 15) ^ row) << 4));
            } else if (ch < CS_CHUNKS + p.nkv) {
                const int g = (ch - CS_CHUNKS) * 64 + lane;
                const int row = g / p.pitch_g, col = g - row * p.pitch_g;
                if (row < TILE_TOK && col < p.row_g) off = (uint32_t)(row * (int)p.c_s1 + col * 16);
            }
        }
        doff[i] = off;
    }
    __syncthreads();

    float* sp = &s_part[wave][0];
    uint16_t* spp = &s_p[wave][0];
    uint16_t* spl = &s_plo[FMT == FMT_BF16 ? wave : 0][0];
    float* salpha = &s_alpha[wave][0];
    cur_first(st.cc, P, p.n, st.beg, st.end);
    st.ld = st.cc;
    st.j = 0;
    st.new_seg = true;
    dma_page<NLD>(p, st.ld, P, s_x0, wave, doff);
    cur_next(st.ld, P, p.n, st.beg, st.end);
    dma_page<NLD>(p, st.ld, P, s_x1, wave, doff);
    if (st.ld.valid) cur_next(st.ld, P, p.n, st.beg, st.end);

    half8_t ab[MTV][4];
    f32x4_t acc[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) acc[k] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    while (true) {
        if (!decode_iter<FMT, MTV, NB, NLD>(st, wt, ab, acc, sm, doff, kpack, s_x0, s_x2, sp, spp, spl, salpha,
                                            s_kmask, &s_qh[wave][0], lane, wave))
            break;
        if (!decode_iter<FMT, MTV, NB, NLD>(st, wt, ab, acc, sm, doff, kpack, s_x1, s_x0, sp, spp, spl, salpha,
                                            s_kmask, &s_qh[wave][0], lane, wave))
            break;
        if (!decode_iter<FMT, MTV, NB, NLD>(st, wt, ab, acc, sm, doff, kpack, s_x2, s_x1, sp, spp, spl, salpha,
                                            s_kmask, &s_qh[wave][0], lane, wave))
            break;
    }
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): no copy may land after the workgroup ends
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

template <int FMT, int MTV, int XB, int NLD>
static const void* pick_nb(int nb) {
    if (nb <= 1) return (const void*)&decode_kernel<FMT, MTV, 1, XB, NLD>;
    if (nb <= 2) return (const void*)&decode_kernel<FMT, MTV, 2, XB, NLD>;
    return (const void*)&decode_kernel<FMT, MTV, 4, XB, NLD>;
}

// Rank tiles per wave held in VGPRs: the wave plan balances whole heads to within a
// tile of TT / 8, so MTV = ceil(TT / 8) covers every wave for the usual rank mixes (a
// wave with more streams the rest of its tiles from L2).
template <int FMT, int XB, int NLD>
static int launch_decode(const DecodeParams& p, int nb, int grid, hipStream_t stream) {
    const int need = (p.TT + NWAVE - 1) / NWAVE;
    const void* fn = need <= 4 ? pick_nb<FMT, 4, XB, NLD>(nb)
                     : need <= 8 ? pick_nb<FMT, 8, XB, NLD>(nb)
                     : need <= 9 ? pick_nb<FMT, 9, XB, NLD>(nb)
                                 : pick_nb<FMT, 10, XB, NLD>(nb);
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(grid), dim3(NTHR), args, 0, stream));
    return STARKV_OK;
}

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
    p.pitch_g = p.row_g | 1;
    p.pitch_b = p.pitch_g * 16;
    p.nkv = (TILE_TOK * p.pitch_g + 63) / 64;
    if (fmt == FMT_Q4) {
        const int nch = CS_CHUNKS + p.nkv;
        SKV_CHECK(nch <= NLD_Q4 * NWAVE && nch * 1024 <= XB_Q4,
                  "decode: a page needs %d KB of LDS (> %d): row %d bytes is too wide", nch, NLD_Q4 * NWAVE,
                  row_bytes);
    } else {
        SKV_CHECK(lowrank_copies(p.k_width, nb) > 0,
                  "decode: a page of k_width %d and v_rank %d needs more than 48 KB of LDS per buffer", p.k_width,
                  a.v_rank);
        p.nch = lowrank_chunks(p.k_width, nb);
        p.lds_bytes = lowrank_lds_bytes(p.k_width, nb);
    }
    p.ws = (uint8_t*)a.ws;
    p.ws_tiles = wl.tiles; p.ws_plan = wl.plan; p.ws_ab = wl.ab;
    p.ws_m = wl.m; p.ws_l = wl.l; p.ws_acc = wl.acc;

    hipLaunchKernelGGL(setup_kernel, dim3(1), dim3(1024), 0, stream, a.seq_lens, a.n, a.max_seq_len, a.grid, a.Hq,
                       a.Hkv, TT, a.k_ranks, a.k_offsets, a.t_head, a.t_nout, a.t_last, p.ws, wl.tiles, wl.plan);
    SKV_HIP(hipGetLastError());
    hipLaunchKernelGGL(fold_tiles_kernel, dim3((TT * 128 + 255) / 256, a.n), dim3(256), 0, stream, a.q, a.q_s0,
                       a.q_s1, a.q_dt, a.k_up, a.ku_s0, a.w_dt, (const uint8_t*)p.ws + wl.tiles, TT,
                       a.scale * LOG2E, fmt == FMT_Q4 ? 1 : 0, p.ws + wl.ab);
    SKV_HIP(hipGetLastError());
    const bool timed = g_prof.on && 2 * g_prof.used + 1 < (int)g_prof.ev.size();
    if (timed) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used], stream));
    int rc = fmt == FMT_Q4 ? launch_decode<FMT_Q4, XB_Q4, NLD_Q4>(p, nb, a.grid, stream)
                           : launch_lowrank(p, fmt, nb, a.grid, stream);
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
