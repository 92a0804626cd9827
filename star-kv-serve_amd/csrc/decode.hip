// Paged decode over the STAR-KV low-rank cache, bf16/fp16 codes and 3.2-bit codes.
//
// Math (per request b, query head h, token l):
//   logit = scale * q . RoPE_l(U_h^T x_l)            paged_decode.py:31-102 / paged_quant.py:258-304
//         = sum_r x_l[r] * ([cos_l | sin_l] . AB[r])  AB = q folded into U (paged_quant.py:241-255,
//                                                      kv_quant.py:42-50)
//   out   = (softmax(logit) @ V_codes) @ v_up_by_q[h]  paged_decode.py:105-147, 220-226
//
// MI355X design, four launches per call (all grids are functions of host ints):
// 1. setup: the per-16-lane rank-tile table and the prefix sums of the request
//    lengths, into the workspace.
// 2. fold: AB for every (request, rank tile) in fp16, written in the A-operand lane
//    order of v_mfma_f32_16x16x32_f16, so the decode kernel loads it straight into
//    its final registers.
// 3. decode: one persistent workgroup (8 waves) per CU. The requests' tokens are laid
//    end to end and cut into `grid` equal contiguous ranges, so every workgroup
//    streams the same number of cache rows whatever the lengths are; a range that
//    crosses a request boundary emits one split-K partial per request. A tile is one
//    16-token page; whole rows are copied global->LDS with 16-byte LDS-DMA loads,
//    three pages in flight. The current request's AB lives in VGPRs (each wave holds
//    a contiguous slice of rank tiles); z = AB . [cos|sin]^T runs on MFMA with the
//    page's 16 positions as N, and each lane multiplies its 4 z values by its 4 codes
//    (bf16/fp16, or unpacked nibbles). Per-tile partials meet in LDS, an online
//    softmax per (head, token) follows, then P[H, 16] @ V[16, r_v] on
//    v_mfma_f32_32x32x16 with the accumulator kept in LDS.
// 4. merge: per (request, head) log-sum-exp of the partials, then the lift through
//    v_up_by_q.
#include <stdio.h>

#include <vector>

#include "common.hpp"

namespace starkv {

enum { FMT_BF16 = 0, FMT_F16 = 1, FMT_Q4 = 2 };

constexpr int NWAVE = 8;
constexpr int NTHR = NWAVE * 64;
constexpr int TILE_TOK = 16;
constexpr int MAX_REQ_PER_CALL = 1024;
constexpr float LOG2E = 1.4426950408889634f;
constexpr int AB_TILE_BYTES = 4 * 64 * 16;  // 4 K-steps x 64 lanes x 8 fp16
constexpr int AB_SLACK_TILES = 16;
constexpr int MAX_TT = 96;                   // rank tiles per call (W <= 1536 for MHA)           // a wave may read up to 10 tiles past its range

// Workspace layout, in bytes from the base (every region 256-byte aligned):
//   hdr    int   [2 + n]      S (tokens per workgroup), P[0..n] (prefix of clamped lengths)
//   tiles  int4  [TT]         {q head, first cache lane, valid | nout << 8 | last << 16, kv head}
//   htile  int2  [Hq]         {first tile, tiles} per query head
//   ab     fp16  [n][TT][4][64][8]
//   m, l   fp32  [slots][Hq]  (log2-domain running max and sum per partial)
//   acc    fp32  [slots][Hq][v_rank]
struct WsLayout {
    size_t hdr, tiles, htile, ab, m, l, acc, total;
};

static inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

static WsLayout ws_layout(int n, int Hq, int TT, int v_rank, int grid) {
    WsLayout w;
    const size_t slots = (size_t)grid + n;
    size_t o = 0;
    w.hdr = o; o = al256(o + (size_t)(n + 2) * 4);
    w.tiles = o; o = al256(o + (size_t)TT * 16);
    w.htile = o; o = al256(o + (size_t)Hq * 8);
    w.ab = o; o = al256(o + ((size_t)n * TT + AB_SLACK_TILES) * AB_TILE_BYTES);
    w.m = o; o = al256(o + slots * Hq * 4);
    w.l = o; o = al256(o + slots * Hq * 4);
    w.acc = o; o = al256(o + slots * Hq * (size_t)v_rank * 4);
    w.total = o;
    return w;
}

struct DecodeParams {
    const uint8_t* cache; int64_t c_s0, c_s1;      // bytes
    int block_size;
    const int32_t* bt; int64_t bt_s0, bt_s1;
    int n, Hq, TT, k_width, v_rank;
    int ks_off, vs_off, vq_off, v_nout, v_nbo;     // QuantRow (3.2-bit)
    int row_g, pitch_g, kv_bytes;                  // LDS staging geometry (granules of 16 bytes)
    int ngr, nld;                                  // granules per page (rows + cos/sin), copies per wave
    float inv_pitch;
    const uint8_t* cs; int64_t cs_s0b; int cs_dt;  // cos/sin table, row stride in bytes, 2-byte dtype
    uint8_t* ws;
    size_t ws_tiles, ws_htile, ws_ab, ws_m, ws_l, ws_acc;
    int slots, units, ncol_t, hpad;
};

__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------------------
// 1. setup: tile table + prefix sums. One workgroup of 1024 threads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void setup_kernel(const int32_t* __restrict__ seq_lens, int n, int max_seq_len,
                                                     int grid, int Hq, int Hkv, int TT,
                                                     const int32_t* __restrict__ k_ranks,
                                                     const int32_t* __restrict__ k_offsets,
                                                     const int32_t* __restrict__ t_head,
                                                     const int32_t* __restrict__ t_nout,
                                                     const int32_t* __restrict__ t_last, uint8_t* __restrict__ ws,
                                                     size_t ws_tiles, size_t ws_htile) {
    __shared__ int s_wsum[16];
    __shared__ int s_total;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int* hdr = (int*)ws;
    int4* tiles = (int4*)(ws + ws_tiles);
    int2* htile = (int2*)(ws + ws_htile);

    // Prefix sums of min(max(seq_len, 0), max_seq_len) over n <= 1024 requests.
    const int a = tid < n ? min(max(seq_lens[tid], 0), max_seq_len) : 0;
    int s = a;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(s, o, 64);
        if (lane >= o) s += y;
    }
    if (lane == 63) s_wsum[wave] = s;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; ++w) off += s_wsum[w];
    if (tid < n) hdr[2 + tid] = off + s;
    if (tid == 0) hdr[1] = 0;
    if (tid == 1023) s_total = off + s;
    __syncthreads();
    if (tid == 0) hdr[0] = (s_total + grid - 1) / grid;

    // Tile table.
    if (t_head) {  // 3.2-bit: the k_tables arrays, lanes contiguous, MHA
        for (int t = tid; t < TT; t += blockDim.x)
            tiles[t] = make_int4(t_head[t], 16 * t, 16 | (t_nout[t] << 8) | ((t_last[t] != 0) << 16), t_head[t]);
        if (tid < Hq) {
            int first = -1, cnt = 0;
            for (int t = 0; t < TT; ++t)
                if (t_head[t] == tid) { if (first < 0) first = t; ++cnt; }
            htile[tid] = make_int2(first < 0 ? 0 : first, cnt);
        }
    } else if (tid < Hq) {  // bf16/fp16: ceil(rank / 16) tiles per query head, kv = h / group
        const int grp = Hq / Hkv;
        int t0 = 0;
        for (int h = 0; h < tid; ++h) t0 += (k_ranks[h / grp] + 15) >> 4;
        const int kv = tid / grp, R = k_ranks[kv], o = k_offsets[kv];
        const int nt = (R + 15) >> 4;
        int cnt = 0;
        for (int j = 0; j < nt && t0 + j < TT; ++j, ++cnt)
            tiles[t0 + j] = make_int4(tid, o + 16 * j, min(16, R - 16 * j) | ((j == nt - 1) << 16), kv);
        htile[tid] = make_int2(min(t0, TT), cnt);
    }
}

// ---------------------------------------------------------------------------
// 2. fold: AB[b][t][ks][lane] = 8 fp16 of row r = tile lane0 + (lane & 15), columns
//    32 ks + 8 (lane >> 4) .. +8, scaled by scale*log2(e); rows past the head's
//    rank are zero (paged_decode.py:79-81 masks them).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fold_tiles_kernel(const void* __restrict__ q, int64_t q_s0, int64_t q_s1,
                                                         int q_dt, const void* __restrict__ k_up, int64_t ku_s0,
                                                         int ku_dt, const uint8_t* __restrict__ ws_tiles_p, int TT,
                                                         float sc, uint8_t* __restrict__ ab) {
    const int b = blockIdx.y;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // (tile, k2, lane)
    const int t = idx >> 7, k2 = (idx >> 6) & 1, lane = idx & 63;
    if (t >= TT) return;
    const int4 tm = ((const int4*)ws_tiles_p)[t];
    const int lr = lane & 15, lg = lane >> 4;
    const int c0 = 32 * k2 + 8 * lg;
    const int64_t ur = (int64_t)(tm.y + lr) * ku_s0;
    const int64_t qh = (int64_t)b * q_s0 + (int64_t)tm.x * q_s1;
    const float s = lr < (tm.z & 255) ? sc : 0.f;
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
// Token cursor: which (request, page) a workgroup visits next. P (the prefix of
// the clamped lengths) is read with scalar loads from the workspace header.
// ---------------------------------------------------------------------------
typedef const __attribute__((address_space(4))) int32_t* cint_p;

struct Cursor {
    int b, k, lo, hi;  // request, page, request-local token range [lo, hi) of this workgroup
    bool valid;
};

__device__ __forceinline__ void cur_set(Cursor& c, cint_p P, int beg, int end) {
    const int pb = P[c.b];
    c.lo = max(beg, pb) - pb;
    c.hi = min(end, P[c.b + 1]) - pb;
    c.k = c.lo / TILE_TOK;
}

__device__ __forceinline__ void cur_first(Cursor& c, cint_p P, int n, int beg, int end) {
    int lo = 0, hi = n - 1;  // largest b with P[b] <= beg; then P[b + 1] > beg
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (P[mid] <= beg) lo = mid; else hi = mid - 1;
    }
    c.b = lo;
    c.valid = beg < end;
    if (c.valid) cur_set(c, P, beg, end);
}

// Returns true when the next tile starts a new request (the current one ended).
__device__ __forceinline__ bool cur_next(Cursor& c, cint_p P, int n, int beg, int end) {
    if (TILE_TOK * (c.k + 1) < c.hi) {
        ++c.k;
        return false;
    }
    int b = c.b + 1;
    while (b < n && P[b + 1] == P[b]) ++b;
    if (b >= n || P[b] >= end) {
        c.valid = false;
        return true;
    }
    c.b = b;
    cur_set(c, P, beg, end);
    return true;
}

// ---------------------------------------------------------------------------
// Global -> LDS copy of one page with 16-byte LDS-DMA loads: the 16 token rows at
// a pitch of pitch_g granules (odd, so rows fall on different banks; granules past
// row_g are filler), then the page's 16 cos/sin rows at a pitch of 17 granules.
// Every wave issues exactly nld copies (surplus ones land in `dummy`), so one
// vmcnt value covers a page on every wave.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dma_page(const DecodeParams& p, const Cursor& c, cint_p P, uint8_t* buf,
                                         uint8_t* dummy, int wave, int lane) {
    const int64_t tok0 = (int64_t)TILE_TOK * c.k;
    const int blk = ((cint_p)p.bt)[c.b * p.bt_s0 + (tok0 / p.block_size) * p.bt_s1];
    const uint8_t* page = p.cache + (int64_t)blk * p.c_s0 + (tok0 % p.block_size) * p.c_s1;
    const int last = P[c.b + 1] - P[c.b] - 1;  // clamp positions to the request's last token
    const int kvg = TILE_TOK * p.pitch_g;
    const int ln = opaque(lane);
    for (int i = 0; i < p.nld; ++i) {
        const int ch = i * NWAVE + wave;
        const int q = ch * 64 + ln;
        const uint8_t* src;
        if (q < kvg) {
            const int row = (int)(((float)q + 0.5f) * p.inv_pitch);
            const int gr = q - row * p.pitch_g;
            src = page + row * p.c_s1 + (gr < p.row_g ? gr * 16 : 0);
        } else {
            const int qc = min(q - kvg, 16 * 17 - 1);
            const int row = qc / 17, gr = qc - row * 17;
            const int64_t pos = min(tok0 + row, (int64_t)last);
            src = p.cs + pos * p.cs_s0b + (gr < 16 ? gr * 16 : 0);
        }
        uint8_t* dst = ch * 64 < p.ngr ? buf + ch * 1024 : dummy;
        if (q >= p.ngr) src = p.cs;  // surplus lanes: any readable address
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    }
}

__device__ __forceinline__ int4 load_tile(cint_p tiles, int t) {
    return make_int4(tiles[4 * t], tiles[4 * t + 1], tiles[4 * t + 2], tiles[4 * t + 3]);
}

// One rank tile: z = AB_tile . cs^T (16 ranks x 16 tokens) and the lane's 4-code product,
// reduced over the 4 row groups; lanes 0..15 write the tile's per-token partial(s).
template <int FMT>
__device__ __forceinline__ void tile_product(const half8_t* a, const half8_t* csb, const uint8_t* xrow, int4 tm,
                                             int lane, int lg, float* s_spart, int tile) {
    f32x4_t z = {0.f, 0.f, 0.f, 0.f};
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], csb[0], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], csb[1], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2], csb[2], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[3], csb[3], z, 0, 0, 0);
    if (FMT == FMT_Q4) {
        // 4 nibbles: lanes x_off + 4 lg .. +4 of token (lane & 15); outlier and inlier sums.
        const uint32_t w = *(const uint16_t*)(xrow + (tm.y >> 1) + 2 * lg);
        const int cnt = min(max(((tm.z >> 8) & 255) - 4 * lg, 0), 4);
        float d = 0.f, dout = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = ((float)((w >> (4 * e)) & 15u) - 8.f) * z[e];
            d += v;
            dout += e < cnt ? v : 0.f;
        }
        float din = d - dout;
        din += __shfl_xor(din, 16, 64);
        dout += __shfl_xor(dout, 16, 64);
        din += __shfl_xor(din, 32, 64);
        dout += __shfl_xor(dout, 32, 64);
        // Lanes 16..63 hold copies of lanes 0..15: they write into the dummy slot.
        ((float2*)s_spart)[(lane < 16 ? tile : MAX_TT + 1) * 16 + (lane & 15)] = make_float2(din, dout);
    } else {
        const uint2 w = *(const uint2*)(xrow + 2 * (tm.y + 4 * lg));
        float x0, x1, x2, x3;
        if (FMT == FMT_BF16) {
            x0 = __uint_as_float(w.x << 16); x1 = __uint_as_float(w.x & 0xffff0000u);
            x2 = __uint_as_float(w.y << 16); x3 = __uint_as_float(w.y & 0xffff0000u);
        } else {
            _Float16 h[4];
            uint32_t ww[2] = {w.x, w.y};
            memcpy(h, ww, 8);
            x0 = (float)h[0]; x1 = (float)h[1]; x2 = (float)h[2]; x3 = (float)h[3];
        }
        float v = x0 * z[0] + x1 * z[1] + x2 * z[2] + x3 * z[3];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        // Lanes 16..63 hold copies of lanes 0..15: they write into the dummy slot.
        s_spart[(lane < 16 ? tile : MAX_TT + 1) * 16 + (lane & 15)] = v;
    }
}

constexpr int MAX_HPAD = 64;     // query heads, padded to the PV MFMA's 32
constexpr int XB_LOWRANK = 48 * 1024;
constexpr int XB_Q4 = 24 * 1024;

struct LoopState {
    Cursor cc, ld;
    int issued, j, beg, end, S, g;
    bool new_seg;
};

// ---------------------------------------------------------------------------
// One page of the decode loop. XC holds the page being computed (its copies were
// issued two pages ago); XN receives the page two ahead. Distinct __shared__
// arrays per buffer let the compiler see that reads of XC never alias the copies
// still in flight, so no vmcnt(0) is inserted before them.
// ---------------------------------------------------------------------------
template <int FMT, int MT>
__device__ __forceinline__ bool decode_page(const DecodeParams& p, LoopState& st, half8_t (&ab)[MT][4],
                                            f32x16_t& acc, const uint8_t* XC, uint8_t* XN, uint8_t* dummy,
                                            float* s_spart, uint16_t* s_p, uint16_t* s_plo, float* s_alpha,
                                            float* s_m, float* s_l,
                                            const int2* s_htile, int tid, int lane, int wave, int ts, int ntw) {
    if (!st.cc.valid) return false;
    cint_p P = (cint_p)(p.ws + 4);
    cint_p tiles = (cint_p)(p.ws + p.ws_tiles);
    const int lr = lane & 15, lg = lane >> 4;
    const Cursor cc = st.cc;
    const int tok0 = TILE_TOK * cc.k;
    const half8_t* ab_base = (const half8_t*)(p.ws + p.ws_ab + ((size_t)cc.b * p.TT + ts) * AB_TILE_BYTES);
    if (st.new_seg) {
        // Tiles past this wave's range load whatever follows (the AB region has slack
        // for it); their products go to a dummy slot.
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ab[i][ks] = ab_base[(i * 4 + ks) * 64 + lane];
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): AB is in registers
    }

    // B1: this page is in LDS for every wave (each waited for its own copies).
    wait_vmcnt_lgkm0(st.issued > st.j + 1 ? p.nld : 0);
    lds_barrier();
    if (st.ld.valid) {
        dma_page(p, st.ld, P, XN, dummy, wave, lane);
        ++st.issued;
        cur_next(st.ld, P, p.n, st.beg, st.end);
    }

    // Cos/sin B operand: lane (lr, lg) holds position tok0 + lr, K elements 32 ks + 8 lg .. +8.
    half8_t csb[4];
    {
        const uint8_t* csr = XC + p.kv_bytes + lr * (17 * 16) + 16 * lg;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint4 w = *(const uint4*)(csr + 64 * ks);
            if (p.cs_dt == STARKV_F16) {
                memcpy(&csb[ks], &w, 16);
            } else {
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    csb[ks][2 * e] = (_Float16)__uint_as_float(ww[e] << 16);
                    csb[ks][2 * e + 1] = (_Float16)__uint_as_float(ww[e] & 0xffff0000u);
                }
            }
        }
    }

    // ---- K side ---------------------------------------------------------------
    const uint8_t* xrow = XC + lr * p.pitch_g * 16;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int t = i < ntw ? ts + i : MAX_TT;  // MAX_TT: the dummy slot
        tile_product<FMT>(ab[i], csb, xrow, load_tile(tiles, min(ts + i, p.TT - 1)), lane, lg, s_spart, t);
    }
    for (int i = MT; i < ntw; ++i) {
        half8_t a[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) a[ks] = ab_base[(i * 4 + ks) * 64 + lane];
        tile_product<FMT>(a, csb, xrow, load_tile(tiles, ts + i), lane, lg, s_spart, ts + i);
    }
    wait_lgkm0_barrier();  // B2: partial logits complete

    // ---- softmax (log2 domain; the scale is folded into AB) -------------------
    for (int idx = tid; idx < p.Hq * TILE_TOK; idx += NTHR) {
        const int h = idx >> 4, r = idx & 15;
        const int tok = tok0 + r;
        const int2 ht = s_htile[h];
        float s = -INFINITY;
        if (tok >= cc.lo && tok < cc.hi) {
            if (FMT == FMT_Q4) {
                const uint32_t sw = *(const uint32_t*)(XC + r * p.pitch_g * 16 + p.ks_off + 4 * h);
                const float so = __uint_as_float(sw << 16), si = __uint_as_float(sw & 0xffff0000u);
                float din = 0.f, dout = 0.f;
                for (int t = ht.x; t < ht.x + ht.y; ++t) {
                    const float2 v = ((const float2*)s_spart)[t * 16 + r];
                    din += v.x;
                    dout += v.y;
                }
                s = si * din + so * dout;
            } else {
                s = 0.f;
                for (int t = ht.x; t < ht.x + ht.y; ++t) s += s_spart[t * 16 + r];
            }
        }
        const float m_old = s_m[h];
        const float m_new = fmaxf(m_old, row16_max(s));
        const float pe = exp2f(s - m_new);
        const float alpha = exp2f(m_old - m_new);
        const float psum = row16_sum(pe);
        if (r == 0) {
            s_m[h] = m_new;
            s_l[h] = s_l[h] * alpha + psum;
            s_alpha[h] = alpha;
        }
        if (FMT == FMT_BF16) {
            // P = hi + lo in two bfloat16 parts: the PV product keeps ~16 bits of P.
            const uint16_t hi = f32_to_bf16_rne(pe);
            s_p[idx] = hi;
            s_plo[idx] = f32_to_bf16_rne(pe - __uint_as_float((uint32_t)hi << 16));
        } else {
            _Float16 hv = (_Float16)pe;
            uint16_t u;
            memcpy(&u, &hv, 2);
            s_p[idx] = u;
        }
    }
    wait_lgkm0_barrier();  // B3: P and alpha complete

    // ---- PV: acc[32 heads, 32 cols] = alpha * acc + P[32, 16] @ V[16, 32] -------
    if (wave < p.units) {
        const int ln = opaque(lane);
        const int hb = wave / p.ncol_t, ct = wave % p.ncol_t;
        const int c = ct * 32 + (ln & 31);
        const int kh = ln >> 5;  // tokens 8 kh .. 8 kh + 7
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4_t al = *(const f32x4_t*)(s_alpha + hb * 32 + 8 * q4 + 4 * kh);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[4 * q4 + e] *= al[e];
        }
        const uint4 pa = *(const uint4*)(s_p + (hb * 32 + (ln & 31)) * 16 + 8 * kh);
        uint32_t bw[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            uint32_t hw[2];
#pragma unroll
            for (int e1 = 0; e1 < 2; ++e1) {
                const int t = 8 * kh + 2 * e2 + e1;
                const int tok = tok0 + t;
                const uint8_t* rowp = XC + t * p.pitch_g * 16;
                uint32_t bits = 0;
                if (tok >= cc.lo && tok < cc.hi && c < p.v_rank) {
                    if (FMT == FMT_Q4) {
                        const bool o = c < p.v_nout;
                        const int ci = o ? c : c - p.v_nout;
                        const int byte = p.vq_off + (o ? 0 : p.v_nbo) + (ci >> 1);
                        const uint32_t nib = (rowp[byte] >> (4 * (ci & 1))) & 15u;
                        const uint32_t sw = *(const uint32_t*)(rowp + p.vs_off);
                        const float sc = o ? __uint_as_float(sw << 16) : __uint_as_float(sw & 0xffff0000u);
                        _Float16 hv = (_Float16)(((float)nib - 8.f) * sc);
                        uint16_t u;
                        memcpy(&u, &hv, 2);
                        bits = u;
                    } else {
                        bits = *(const uint16_t*)(rowp + 2 * (p.k_width + c));
                    }
                }
                hw[e1] = bits;
            }
            bw[e2] = hw[0] | (hw[1] << 16);
        }
        uint32_t aw[4] = {pa.x, pa.y, pa.z, pa.w};
        if (FMT == FMT_BF16) {
            const uint4 pl = *(const uint4*)(s_plo + (hb * 32 + (ln & 31)) * 16 + 8 * kh);
            uint32_t lw[4] = {pl.x, pl.y, pl.z, pl.w};
            bf16x8_t a, al, b;
            memcpy(&a, aw, 16);
            memcpy(&al, lw, 16);
            memcpy(&b, bw, 16);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b, acc, 0, 0, 0);
        } else {
            half8_t a, b;
            memcpy(&a, aw, 16);
            memcpy(&b, bw, 16);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
        }
    }

    // ---- end of this request's range: write the partial, reset ----------------
    Cursor nx = cc;
    const bool seg_end = cur_next(nx, P, p.n, st.beg, st.end);
    if (seg_end) {
        const int slot = cc.b + st.g;
        float* wm = (float*)(p.ws + p.ws_m) + (int64_t)slot * p.Hq;
        float* wl = (float*)(p.ws + p.ws_l) + (int64_t)slot * p.Hq;
        float* wa = (float*)(p.ws + p.ws_acc) + (int64_t)slot * p.Hq * p.v_rank;
        for (int h = tid; h < p.Hq; h += NTHR) {
            wm[h] = s_m[h];
            wl[h] = s_l[h];
        }
        if (wave < p.units) {
            const int ln = opaque(lane);
            const int hb = wave / p.ncol_t, ct = wave % p.ncol_t;
            const int c = ct * 32 + (ln & 31);
            const int kh = ln >> 5;
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const int h = hb * 32 + 8 * (jj >> 2) + 4 * kh + (jj & 3);
                if (h < p.Hq && c < p.v_rank) wa[(int64_t)h * p.v_rank + c] = acc[jj];
                acc[jj] = 0.f;
            }
        }
        wait_lgkm0_barrier();  // every read of m and l is done before the reset
        for (int h = tid; h < p.Hq; h += NTHR) {
            s_m[h] = -INFINITY;
            s_l[h] = 0.f;
        }
    }
    st.cc = nx;
    st.new_seg = seg_end;
    ++st.j;
    return true;
}

// ---------------------------------------------------------------------------
// 3. decode. MT = rank tiles per wave held in VGPRs; a wave with more tiles reads
//    the rest from the workspace (L2) on every page. XB = bytes per page buffer.
// ---------------------------------------------------------------------------
template <int FMT, int MT, int XB>
__global__ __launch_bounds__(NTHR) void decode_kernel(const DecodeParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t s_x0[XB];
    __shared__ __attribute__((aligned(16))) uint8_t s_x1[XB];
    __shared__ __attribute__((aligned(16))) uint8_t s_x2[XB];
    __shared__ __attribute__((aligned(16))) uint8_t s_dummy[1024];
    __shared__ __attribute__((aligned(16))) float s_spart[(MAX_TT + 2) * TILE_TOK * (FMT == FMT_Q4 ? 2 : 1)];
    __shared__ __attribute__((aligned(16))) uint16_t s_p[MAX_HPAD * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_plo[FMT == FMT_BF16 ? MAX_HPAD * TILE_TOK : 8];
    __shared__ __attribute__((aligned(16))) float s_alpha[MAX_HPAD];
    __shared__ float s_m[MAX_HPAD];
    __shared__ float s_l[MAX_HPAD];
    __shared__ int2 s_htile[MAX_HPAD];

    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    for (int h = tid; h < p.Hq; h += NTHR) {
        s_htile[h] = ((const int2*)(p.ws + p.ws_htile))[h];
        s_m[h] = -INFINITY;
        s_l[h] = 0.f;
    }
    for (int h = tid; h < p.hpad; h += NTHR) s_alpha[h] = 1.f;
    for (int i = tid; i < p.hpad * TILE_TOK; i += NTHR) {
        s_p[i] = 0;
        if (FMT == FMT_BF16) s_plo[i] = 0;
    }
    __syncthreads();

    cint_p P = (cint_p)(p.ws + 4);
    LoopState st;
    st.g = blockIdx.x;
    st.S = ((cint_p)p.ws)[0];
    const int T = P[p.n];
    st.beg = min(st.g * st.S, T);
    st.end = min(st.beg + st.S, T);
    if (st.beg >= st.end) return;

    const int ts = (wave * p.TT) / NWAVE, ntw = ((wave + 1) * p.TT) / NWAVE - ts;
    cur_first(st.cc, P, p.n, st.beg, st.end);
    st.ld = st.cc;
    st.issued = 0;
    st.j = 0;
    st.new_seg = true;
    dma_page(p, st.ld, P, s_x0, s_dummy, wave, lane);
    ++st.issued;
    cur_next(st.ld, P, p.n, st.beg, st.end);
    if (st.ld.valid) {
        dma_page(p, st.ld, P, s_x1, s_dummy, wave, lane);
        ++st.issued;
        cur_next(st.ld, P, p.n, st.beg, st.end);
    }

    half8_t ab[MT][4];
    f32x16_t acc = {};
    while (true) {
        if (!decode_page<FMT, MT>(p, st, ab, acc, s_x0, s_x2, s_dummy, s_spart, s_p, s_plo, s_alpha, s_m, s_l,
                                  s_htile, tid,
                                  lane, wave, ts, ntw))
            break;
        if (!decode_page<FMT, MT>(p, st, ab, acc, s_x1, s_x0, s_dummy, s_spart, s_p, s_plo, s_alpha, s_m, s_l,
                                  s_htile, tid,
                                  lane, wave, ts, ntw))
            break;
        if (!decode_page<FMT, MT>(p, st, ab, acc, s_x2, s_x1, s_dummy, s_spart, s_p, s_plo, s_alpha, s_m, s_l,
                                  s_htile, tid,
                                  lane, wave, ts, ntw))
            break;
    }
}

// ---------------------------------------------------------------------------
// 4. merge: per (request, head) combine the partials (log2-domain LSE), then lift.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(128) void merge_kernel(const uint8_t* __restrict__ ws, size_t ws_m, size_t ws_l,
                                                    size_t ws_acc, int Hq, int v_rank, const void* __restrict__ vup,
                                                    int64_t vu_s0, int64_t vu_s1, int w_dt, void* __restrict__ out,
                                                    int64_t o_s0, int64_t o_s1, int out_dt) {
    extern __shared__ float s_o[];  // [v_rank]
    const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int* hdr = (const int*)ws;
    const int S = hdr[0];
    const int pb = hdr[1 + b], pe = hdr[2 + b];
    if (pe <= pb || S <= 0) {  // no tokens: softmax over an empty row (NaN, as the reference)
        for (int d = tid; d < 128; d += blockDim.x)
            store_f(out, (int64_t)b * o_s0 + (int64_t)h * o_s1 + d, out_dt, __builtin_nanf(""));
        return;
    }
    const int k_lo = pb / S, k_hi = (pe - 1) / S;
    const float* wm = (const float*)(ws + ws_m);
    const float* wl = (const float*)(ws + ws_l);
    const float* wa = (const float*)(ws + ws_acc);
    float M = -INFINITY;
    for (int k = k_lo; k <= k_hi; ++k) M = fmaxf(M, wm[(int64_t)(k + b) * Hq + h]);
    float l = 0.f;
    for (int k = k_lo; k <= k_hi; ++k) {
        const int64_t sl = (int64_t)(k + b) * Hq + h;
        l += wl[sl] * exp2f(wm[sl] - M);
    }
    const float inv_l = 1.f / l;
    for (int c = tid; c < v_rank; c += blockDim.x) {
        float a = 0.f;
        for (int k = k_lo; k <= k_hi; ++k) {
            const int64_t sl = (int64_t)(k + b) * Hq + h;
            a += wa[sl * v_rank + c] * exp2f(wm[sl] - M);
        }
        s_o[c] = a * inv_l;
    }
    __syncthreads();
    for (int d = tid; d < 128; d += blockDim.x) {
        float o = 0.f;
        const int64_t vb = (int64_t)h * vu_s0 + d;
        for (int c = 0; c < v_rank; ++c) o += s_o[c] * load_f(vup, vb + (int64_t)c * vu_s1, w_dt);
        store_f(out, (int64_t)b * o_s0 + (int64_t)h * o_s1 + d, out_dt, o);
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

static int mt_for(int TT) {
    int mt = (TT + NWAVE - 1) / NWAVE;
    if (mt <= 4) return 4;
    if (mt <= 6) return 6;
    if (mt <= 8) return 8;
    return 10;  // beyond 10 tiles per wave the rest stream from L2 each page
}

template <int FMT, int XB>
static int launch_decode(const DecodeParams& p, int mt, int grid, hipStream_t stream) {
    const void* fn = nullptr;
    switch (mt) {
        case 4: fn = (const void*)&decode_kernel<FMT, 4, XB>; break;
        case 6: fn = (const void*)&decode_kernel<FMT, 6, XB>; break;
        case 8: fn = (const void*)&decode_kernel<FMT, 8, XB>; break;
        default: fn = (const void*)&decode_kernel<FMT, 10, XB>; break;
    }
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(grid), dim3(NTHR), args, 0, stream));
    return STARKV_OK;
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
    SKV_CHECK(a.Hq >= 1 && a.Hq <= MAX_HPAD, "decode: num_heads=%d (1..%d)", a.Hq, MAX_HPAD);
    SKV_CHECK(a.max_seq_len >= 1, "decode: max_seq_len must be >= 1");
    SKV_CHECK(a.v_rank >= 1, "decode: v_rank must be >= 1");
    SKV_CHECK(a.grid >= 1, "decode: grid must be >= 1");
    SKV_CHECK(TT >= 1 && TT <= MAX_TT, "decode: %d rank tiles (1..%d: k_width x heads per kv head <= %d)", TT,
              MAX_TT, MAX_TT * 16);
    const WsLayout wl = ws_layout(a.n, a.Hq, TT, a.v_rank, a.grid);
    SKV_CHECK(a.ws_bytes >= wl.total, "decode: workspace %zu bytes < %zu needed", a.ws_bytes, wl.total);
    SKV_CHECK(((uintptr_t)a.ws % 256) == 0, "decode: workspace must be 256-byte aligned");
    SKV_CHECK(p.block_size % TILE_TOK == 0, "decode: block_size %d must be a multiple of 16", p.block_size);
    SKV_CHECK(((uintptr_t)p.cache % 16) == 0 && p.c_s0 % 16 == 0 && p.c_s1 % 16 == 0,
              "decode: cache base and byte strides must be 16-byte aligned (c_s0=%lld c_s1=%lld)", (long long)p.c_s0,
              (long long)p.c_s1);
    SKV_CHECK(row_bytes % 16 == 0, "decode: cache row (%d bytes) must be a multiple of 16 bytes", row_bytes);
    SKV_CHECK(p.c_s1 >= row_bytes, "decode: slot stride %lld < row bytes %d", (long long)p.c_s1, row_bytes);
    SKV_CHECK(a.cs_dt == STARKV_F16 || a.cs_dt == STARKV_BF16, "decode: cos_sin must be fp16 or bf16");
    SKV_CHECK(a.cs_s0 % 8 == 0 && ((uintptr_t)a.cs % 16) == 0, "decode: cos_sin rows must be 16-byte aligned");
    SKV_CHECK(a.q_s1 % 8 == 0 && a.q_s0 % 8 == 0 && ((uintptr_t)a.q % 16) == 0,
              "decode: query rows must be 16-byte aligned (strides multiples of 8)");
    SKV_CHECK(a.ku_s0 % 8 == 0 && ((uintptr_t)a.k_up % 16) == 0, "decode: k_up rows must be 16-byte aligned");
    const int ncol_t = (a.v_rank + 31) / 32;
    const int hblk = (a.Hq + 31) / 32;
    SKV_CHECK(ncol_t * hblk <= NWAVE, "decode: %d x %d PV tiles exceed %d waves (v_rank %d, heads %d)", hblk, ncol_t,
              NWAVE, a.v_rank, a.Hq);

    p.bt = a.bt; p.bt_s0 = a.bt_s0; p.bt_s1 = a.bt_s1;
    p.n = a.n; p.Hq = a.Hq; p.TT = TT; p.v_rank = a.v_rank;
    p.cs = (const uint8_t*)a.cs; p.cs_s0b = a.cs_s0 * 2; p.cs_dt = a.cs_dt;
    p.row_g = row_bytes / 16;
    p.pitch_g = p.row_g | 1;
    p.inv_pitch = 1.0f / (float)p.pitch_g;
    p.kv_bytes = TILE_TOK * p.pitch_g * 16;
    p.ngr = TILE_TOK * p.pitch_g + TILE_TOK * 17;
    const int nch = (p.ngr + 63) / 64;
    p.nld = (nch + NWAVE - 1) / NWAVE;
    SKV_CHECK(p.nld <= 15, "decode: %d copies per wave per page (row %d bytes) exceeds 15", p.nld, row_bytes);
    const int xb = fmt == FMT_Q4 ? XB_Q4 : XB_LOWRANK;
    SKV_CHECK(nch * 1024 <= xb, "decode: a page needs %d bytes of LDS (> %d): row %d bytes is too wide", nch * 1024,
              xb, row_bytes);
    p.ws = (uint8_t*)a.ws;
    p.ws_tiles = wl.tiles; p.ws_htile = wl.htile; p.ws_ab = wl.ab;
    p.ws_m = wl.m; p.ws_l = wl.l; p.ws_acc = wl.acc;
    p.slots = a.grid + a.n;
    p.ncol_t = ncol_t;
    p.units = ncol_t * hblk;
    p.hpad = hblk * 32;

    hipLaunchKernelGGL(setup_kernel, dim3(1), dim3(1024), 0, stream, a.seq_lens, a.n, a.max_seq_len, a.grid, a.Hq,
                       a.Hkv, TT, a.k_ranks, a.k_offsets, a.t_head, a.t_nout, a.t_last, p.ws, wl.tiles, wl.htile);
    SKV_HIP(hipGetLastError());
    hipLaunchKernelGGL(fold_tiles_kernel, dim3((TT * 128 + 255) / 256, a.n), dim3(256), 0, stream, a.q, a.q_s0,
                       a.q_s1, a.q_dt, a.k_up, a.ku_s0, a.w_dt, (const uint8_t*)p.ws + wl.tiles, TT,
                       a.scale * LOG2E, p.ws + wl.ab);
    SKV_HIP(hipGetLastError());
    const int mt = mt_for(TT);
    const bool timed = g_prof.on && 2 * g_prof.used + 1 < (int)g_prof.ev.size();
    if (timed) SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used], stream));
    int rc = fmt == FMT_Q4 ? launch_decode<FMT_Q4, XB_Q4>(p, mt, a.grid, stream)
             : fmt == FMT_BF16 ? launch_decode<FMT_BF16, XB_LOWRANK>(p, mt, a.grid, stream)
                               : launch_decode<FMT_F16, XB_LOWRANK>(p, mt, a.grid, stream);
    if (rc) return rc;
    SKV_HIP(hipGetLastError());
    if (timed) {
        SKV_HIP(hipEventRecord(g_prof.ev[2 * g_prof.used + 1], stream));
        ++g_prof.used;
    }
    hipLaunchKernelGGL(merge_kernel, dim3(a.n, a.Hq), dim3(128), a.v_rank * 4, stream, (const uint8_t*)p.ws, wl.m,
                       wl.l, wl.acc, a.Hq, a.v_rank, a.vup, a.vu_s0, a.vu_s1, a.w_dt, a.out, a.o_s0, a.o_s1,
                       a.out_dt);
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
    p.block_size = block_size;
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
    p.block_size = block_size;
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
