// Two-pass decode for V ranks too wide for the one-pass kernels (bf16/fp16 codes with
// v_rank > 256, 3.2-bit codes with more than five 64-lane P @ V blocks), and the merge
// of its partials. decode.hip runs, per call: prep, the logits pass (the one-pass
// kernels with NB = 0: K side and softmax statistics only, every valid logit stored in
// the workspace), then `pv_kernel` here, then `merge_wide_kernel` here.
//
// The reference splits its V pass the same way: logits first, then P @ V over
// column blocks of at most 512 (paged_decode.py:105-147, 199-219) or 128 channels
// inside one outlier/inlier block (paged_quant.py:311-354, 390-407).
//
// pv_kernel. The same persistent workgroups and token ranges as the logits pass, so
// that partial slot (request b, workgroup g) = b + g matches the (m, l) the logits pass
// stored for it. Per page of 16 tokens the workgroup copies into LDS, with buffer loads
// that write LDS directly (16 bytes per lane):
//   - the V bytes of the 16 rows: bf16/fp16, the columns [c0, c0 + cw) of this launch's
//     window; 3.2-bit, every V byte (scales, outlier and inlier nibbles);
//   - the 16 logits of every head (2 KB) and the slot's reference max per head.
// Since the reference max of a slot is final, P = exp2(logit - m) needs no rescaling.
// P @ V runs on v_mfma_f32_32x32x16 (M = 32 heads, N = 32 columns, K = the page's 16
// tokens): A = P (bf16 codes: P = hi + lo, two bf16 parts; fp16: P; 3.2-bit: P * s_out
// for outlier blocks and P * s_in for inlier blocks, s the token's V scales, folded as
// paged_quant.py:343-346 does), B = 16 tokens x 32 columns of V read with
// ds_read_b64_tr_b16: a 16-lane group hands in 4 tokens x 16 columns and lane i gets
// column i of the 4 tokens. 3.2-bit V nibbles are first expanded once per page, by
// the whole workgroup, into an fp16 table of (n - 8) in that layout. Wave w owns the
// 32-column blocks w, w + 8, ...; at the end of a request's tokens in the range it
// stores its block of the slot's partial accumulator [Hq][v_rank] (fp32).
//
// LDS. Every 16-byte granule column G (8 code columns) holds the 16 tokens of a page,
// token t in slot t ^ (4 (G & 1)), 256 bytes per granule column, so a page's V (or the
// expanded table) is one 1 KB chunk per 32 columns, and a transposed read of 4 tokens
// x 16 columns by 16 lanes touches 128 distinct bytes per bank group.
#include <algorithm>

#include "decode_pages.hpp"

namespace starkv {

namespace {

constexpr int PV_MAX_DYN_LDS = 160 * 1024 - 1024;  // the kernel's static LDS is a few words

// Swizzled slot of token t in granule column G.
__device__ __forceinline__ int gslot(int G, int t) { return t ^ ((G & 1) << 2); }

typedef short short4v_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v_t* lds_s4p;

// 4 tokens x 16-bit of one column per lane (see the file comment).
__device__ __forceinline__ uint2 tr_read(uint32_t addr) {
    const short4v_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4p)(uintptr_t)addr);
    return __builtin_bit_cast(uint2, r);
}

// Packs 8 fp32 values into 8 bfloat16 (round to nearest even).
__device__ __forceinline__ bf16x8_t to_bf16x8(const float (&v)[8]) {
    bf16x8_t r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)v[e];
    return r;
}
__device__ __forceinline__ half8_t to_f16x8(const float (&v)[8]) {
    half8_t r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)v[e];
    return r;
}

}  // namespace

// Kernel arguments of the P @ V pass (host ints and pointers only).
struct PvParams {
    const uint8_t* cache; int64_t c_s0; int c_s1;  // bytes
    int bs_shift;
    const int32_t* bt; int bt_s0, bt_s1;
    int n, Hq, v_rank;
    int v_off;       // byte of a row where the copied V bytes start (16-aligned)
    int ng;          // 16-byte granules copied per row
    int vs_rel;      // 3.2-bit: V scales at this byte of the copied bytes
    int vq_rel;      // 3.2-bit: first V nibble byte (outlier nibbles), relative
    int v_nout, v_nbo, o32;  // 3.2-bit: outlier columns, their bytes, outlier table columns (v_nout up to 32)
    int c0, ncb;     // window: first (table) column, 32-column blocks
    int nch;         // 1 KB chunks copied per page: V, then logits (2), then the slot's maxima (1)
    int nld;         // copies per wave per page
    int nbuf;        // page buffers in flight (2 or 3)
    int buf_bytes;   // LDS bytes per page buffer (nch KB)
    int tab;         // 3.2-bit: LDS byte of the expanded table
    int lds_bytes;
    uint8_t* ws; size_t ws_plan, ws_m, ws_acc, ws_lg; int lcap;
};

typedef const __attribute__((address_space(4))) PvParams kpv_t;
__device__ __forceinline__ const PvParams& pv_params() {
    kpv_t* pp = (kpv_t*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(pp));
    return *(const PvParams*)pp;
}

// Copy descriptors of one page: its rows, its logits rows (request b, tokens 16 k ..,
// every head), the slot's reference maxima.
struct PvPage {
    int4v_t rv, rl, rm;
};

__device__ __forceinline__ PvPage pv_page_desc(const PvParams& p, const Cursor& c, int blk, int g) {
    PvPage d;
    const bool v = c.valid;
    const int k = v ? c.k : 0;
    const int row0 = (k & ((1 << p.bs_shift) - 1)) * TILE_TOK;
    const uint8_t* page = p.cache + (int64_t)blk * p.c_s0 + (int64_t)row0 * p.c_s1;
    const int rows = v ? min(TILE_TOK, c.len - TILE_TOK * k) : 0;
    d.rv = buffer_rsrc(page, rows * p.c_s1);
    const uint8_t* lg = p.ws + p.ws_lg + ((int64_t)(v ? c.b : 0) * p.Hq * p.lcap + TILE_TOK * k) * 4;
    d.rl = buffer_rsrc(lg, v ? ((p.Hq - 1) * p.lcap + TILE_TOK) * 4 : 0);
    const uint8_t* m = p.ws + p.ws_m + (int64_t)(v ? c.b + g : 0) * p.Hq * 4;
    d.rm = buffer_rsrc(m, v ? ((p.Hq * 4 + 15) & ~15) : 0);
    return d;
}

// The copies of this wave for one page into the buffer at LDS byte `buf`: copy i moves
// chunk 8 i + wave; chunks past nch go to the dummy block and read nothing.
template <int NLD>
__device__ __forceinline__ void pv_copies(const PvParams& p, const PvPage& d, uint32_t buf, uint32_t dummy, int wave,
                                          const uint32_t (&off)[NLD]) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        if (i >= p.nld) break;
        const uint32_t m0 = ch < p.nch ? buf + (uint32_t)ch * 1024u : dummy;
        if (ch < p.nch - 3)
            lds_copy16(d.rv, m0, off[i]);
        else if (ch < p.nch - 1)
            lds_copy16(d.rl, m0, off[i]);
        else
            lds_copy16(d.rm, m0, off[i]);
    }
}

// Expands the 3.2-bit V nibbles of the page in buffer `buf` into the fp16 table of
// (n - 8): table column tc < o32 is outlier column tc (nibbles from vq_rel), else
// inlier column tc - o32 (nibbles from vq_rel + v_nbo); columns past the real ones
// hold whatever bytes follow and are never stored.
__device__ __forceinline__ void pv_expand(const PvParams& p, uint32_t buf, uint32_t tab, int tid) {
    const int items = p.ncb * 4 * TILE_TOK;  // (table granule column, token)
    const int lim = p.ng * 16 - 4;
    for (int it = tid; it < items; it += NTHR) {
        const int TG = it >> 4, t = it & 15;
        const int tc = p.c0 + 8 * TG;
        const int b = tc < p.o32 ? p.vq_rel + (tc >> 1) : p.vq_rel + p.v_nbo + ((tc - p.o32) >> 1);
        // The 4 nibble bytes at b (any alignment): two aligned words, then a funnel shift.
        const int b0 = min(b & ~3, lim), b1 = min((b & ~3) + 4, lim);
        const uint32_t a0 = buf + (uint32_t)((((b0 >> 4) << 4) + gslot(b0 >> 4, t)) * 16 + (b0 & 15));
        const uint32_t a1 = buf + (uint32_t)((((b1 >> 4) << 4) + gslot(b1 >> 4, t)) * 16 + (b1 & 15));
        const uint32_t w0 = lds_ld<uint32_t>(a0), w1 = lds_ld<uint32_t>(a1);
        const uint32_t w = __builtin_amdgcn_alignbyte(w1, w0, (uint32_t)(b & 3));
        uint32_t r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t byte = (w >> (8 * j)) & 0xFFu;
            const uint32_t x = (byte & 0xFu) | ((byte << 12) & 0xF0000u) | 0x64006400u;  // fp16 (1024 + lo, 1024 + hi)
            r[j] = h2_bits(as_h2(x) - (half2_t){(_Float16)1032.f, (_Float16)1032.f});
        }
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        lds_st<u32x4_t>(tab + (uint32_t)((TG * 16 + gslot(TG, t)) * 16), (u32x4_t){r[0], r[1], r[2], r[3]});
    }
}

template <int FMT, int MB, int NLD>
__global__ __launch_bounds__(NTHR) void pv_kernel(const PvParams p0) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_pv[];
    const PvParams& p = pv_params();
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    cint_p P = (cint_p)(p.ws + 4);
    if (((cint_p)(p.ws + p.ws_plan))[NWAVE * PLAN_STRIDE] == 0) return;  // no plan: the merge reports NaN
    const int g = xcd_range(blockIdx.x, gridDim.x);
    const int S_tok = ((cint_p)p.ws)[0];
    const int T = P[p.n];
    const int beg = min(g * S_tok, T), end = min(beg + S_tok, T);
    if (beg >= end) return;

    const uint32_t base = lds_addr(s_pv);
    const uint32_t dummy = base + (uint32_t)(p.lds_bytes - 1024);
    // Buffers start zeroed: rows past a request's end are never copied and must be finite.
    for (int i = tid; i < p.lds_bytes / 16; i += NTHR) ((uint4*)s_pv)[i] = make_uint4(0, 0, 0, 0);

    // Copy offsets of this lane inside a page, per copy i (chunk 8 i + wave).
    uint32_t off[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        uint32_t o = 0x80000000u;  // past every descriptor: no access
        const int nv = p.nch - 3;
        if (ch < nv) {
            const int G = 4 * ch + (lane >> 4), t = gslot(G, lane & 15);
            if (G < p.ng) o = (uint32_t)(t * p.c_s1 + p.v_off + 16 * G);
        } else if (ch < nv + 2) {
            const int h = 16 * (ch - nv) + (lane >> 2);
            if (h < p.Hq) o = (uint32_t)((h * p.lcap) * 4 + 16 * (lane & 3));
        } else if (ch == nv + 2) {
            if (4 * lane < p.Hq) o = (uint32_t)(16 * lane);
        }
        off[i] = o;
    }

    // Lane roles. A operand: head am = lane & 31, tokens 8 ag .. 8 ag + 7 (ag = lane >> 5).
    // B operand (transposed reads): 16-lane group q = lane >> 4 reads tokens 8 (q >> 1) +
    // i / 4 (+ 4), columns 16 (q & 1) + 4 (i % 4) of the block, i = lane & 15.
    const int am = lane & 31, ag = lane >> 5;
    uint32_t trd0, trd1;  // byte offsets of this lane's two transposed reads inside block 0
    {
        const int q = lane >> 4, i = lane & 15;
        const int t = 8 * (q >> 1) + (i >> 2);
        const int col = 16 * (q & 1) + 4 * (i & 3);
        const int G = col >> 3, h = (col >> 2) & 1;
        trd0 = (uint32_t)((G * 16 + gslot(G, t)) * 16 + 8 * h);
        trd1 = (uint32_t)((G * 16 + gslot(G, t + 4)) * 16 + 8 * h);
    }
    const uint32_t lga = (uint32_t)((p.nch - 3) * 1024 + (am * 16 + 8 * ag) * 4);  // logits of (am, 8 ag ..)
    const uint32_t mxa = (uint32_t)((p.nch - 1) * 1024 + am * 4);                   // the slot max of head am
    __syncthreads();

    f32x16_t acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (f32x16_t){};

    Cursor cc, ld;
    cur_first(cc, P, p.n, beg, end);
    ld = cc;
    auto blk_of = [&](const Cursor& c) {
        return c.valid ? ((cint_p)p.bt)[c.b * p.bt_s0 + (c.k >> p.bs_shift) * p.bt_s1] : 0;
    };
    // Prologue: pages 0 .. nbuf - 2 in flight.
    for (int j = 0; j < p.nbuf - 1; ++j) {
        pv_copies<NLD>(p, pv_page_desc(p, ld, blk_of(ld), g), base + (uint32_t)(j * p.buf_bytes), dummy, wave, off);
        if (ld.valid) cur_next(ld, P, p.n, beg, end);
    }
    int jb = 0;  // buffer of the current page
    while (cc.valid) {
        // Page cc is in buffer jb; the copies of the nbuf - 2 pages after it may still run.
        if (p.nbuf == 3)
            wait_vmcnt_lgkm0(p.nld);
        else
            wait_vmcnt_lgkm0(0);
        wait_lgkm0_barrier();  // every wave is done with the previous page's buffer and the table
        {
            const int jn = jb == 0 ? p.nbuf - 1 : jb - 1;  // the buffer the previous page used
            pv_copies<NLD>(p, pv_page_desc(p, ld, blk_of(ld), g), base + (uint32_t)(jn * p.buf_bytes), dummy, wave,
                           off);
            if (ld.valid) cur_next(ld, P, p.n, beg, end);
        }
        const uint32_t buf = base + (uint32_t)(jb * p.buf_bytes);
        uint32_t src = buf;  // where the B operands are read: the page (bf16/fp16) or the table (3.2-bit)
        if (FMT == FMT_Q4) {
            src = base + (uint32_t)p.tab;
            pv_expand(p, buf, src, tid);
            wait_lgkm0_barrier();
        }
        // A operand: P of head am at tokens 8 ag .. 8 ag + 7 of this page.
        const f32x4_t s0 = lds_ld<f32x4_t>(buf + lga), s1 = lds_ld<f32x4_t>(buf + lga + 16);
        const float mx = lds_ld<float>(buf + mxa);
        const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const int tok0 = TILE_TOK * cc.k + 8 * ag;
        float pe[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool ok = am < p.Hq && tok0 + e >= cc.lo && tok0 + e < cc.hi;
            pe[e] = ok ? __builtin_amdgcn_exp2f(sv[e] - mx) : 0.f;
        }
        bf16x8_t ahi, alo;
        half8_t aho, ahi16;
        if (FMT == FMT_BF16) {
            float lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) lo[e] = pe[e] - (float)(__bf16)pe[e];
            ahi = to_bf16x8(pe);
            alo = to_bf16x8(lo);
        } else if (FMT == FMT_F16) {
            aho = to_f16x8(pe);
        } else {
            float po[8], pi[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {  // the token's (outlier, inlier) V scales, bf16
                const int t = 8 * ag + e;
                const uint32_t sw = lds_ld<uint32_t>(buf + (uint32_t)(gslot(0, t) * 16 + p.vs_rel));
                po[e] = pe[e] * __uint_as_float(sw << 16);
                pi[e] = pe[e] * __uint_as_float(sw & 0xffff0000u);
            }
            aho = to_f16x8(po);
            ahi16 = to_f16x8(pi);
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int cb = wave + NWAVE * i;
            if (cb < p.ncb) {
                const uint32_t a = src + (uint32_t)cb * 1024u;
                const uint2 b0 = tr_read(a + trd0), b1 = tr_read(a + trd1);
                const uint4 bw = make_uint4(b0.x, b0.y, b1.x, b1.y);
                if (FMT == FMT_BF16) {
                    const bf16x8_t bv = __builtin_bit_cast(bf16x8_t, bw);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi, bv, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo, bv, acc[i], 0, 0, 0);
                } else {
                    const half8_t bv = __builtin_bit_cast(half8_t, bw);
                    const half8_t av = (FMT == FMT_Q4 && p.c0 + 32 * cb >= p.o32) ? ahi16 : aho;
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i], 0, 0, 0);
                }
            }
        }
        Cursor nx = cc;
        const bool seg_end = cur_next(nx, P, p.n, beg, end);
        if (seg_end) {
            // This lane's column of each of its blocks, for the 16 heads
            // 8 (j / 4) + 4 (lane >> 5) + j % 4 of the 32x32 result.
            const int64_t slot = (int64_t)cc.b + g;
            float* wa = (float*)(p.ws + p.ws_acc) + slot * p.Hq * p.v_rank;
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int cb = wave + NWAVE * i;
                const int tc = p.c0 + 32 * cb + (lane & 31);
                int col = tc;
                if (FMT == FMT_Q4) col = tc < p.o32 ? (tc < p.v_nout ? tc : -1) : p.v_nout + tc - p.o32;
                const bool okc = cb < p.ncb && col >= 0 && col < p.v_rank;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int h = 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
                    if (okc && h < p.Hq) wa[(int64_t)h * p.v_rank + col] = acc[i][j];
                    acc[i][j] = 0.f;
                }
            }
        }
        cc = nx;
        jb = jb + 1 == p.nbuf ? 0 : jb + 1;
    }
    wait_vmcnt_lgkm0(0);  // no copy may land after the workgroup ends
}

// ---------------------------------------------------------------------------
// Merge of the two-pass partials: per (request, head) the log-sum-exp of the slots'
// (m, l), the weighted sum of their accumulators, then the lift through v_up_by_q[h].
// A workgroup takes one head and MW_REQ requests: phase 1 merges request r into LDS
// (wave w takes requests w and w + 4), phase 2 lifts all of them, each thread 8 output
// columns over one sixteenth of the rank columns, and reduces over the sixteenths.
// ---------------------------------------------------------------------------
constexpr int MW_REQ = 8;
constexpr int MW_THR = 256;

static size_t merge_wide_lds(int v_rank) { return (size_t)MW_REQ * v_rank * 4 + (size_t)4 * MW_REQ * 128 * 4; }

template <int DT>
__global__ __launch_bounds__(MW_THR) void merge_wide_kernel(const uint8_t* __restrict__ ws, size_t ws_plan,
                                                            size_t ws_m, size_t ws_l, size_t ws_acc, int n, int Hq,
                                                            int v_rank, const void* __restrict__ vup, int64_t vu_s0,
                                                            int64_t vu_s1, void* __restrict__ out, int64_t o_s0,
                                                            int64_t o_s1, int out_dt) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    float* s_o = (float*)s_dyn;                                    // [MW_REQ][v_rank]
    float* s_red = (float*)(s_dyn + (size_t)MW_REQ * v_rank * 4);  // [4 waves][MW_REQ][128]
    __shared__ int s_live[MW_REQ];
    const int h = blockIdx.x, b0 = blockIdx.y * MW_REQ;  // head in x: a head's workgroups share one XCD's L2
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int* hdr = (const int*)ws;
    const float* wm = (const float*)(ws + ws_m);
    const float* wl = (const float*)(ws + ws_l);
    const float* wa = (const float*)(ws + ws_acc);
    const int S = hdr[0];
    const bool planned = ((const int*)(ws + ws_plan))[NWAVE * PLAN_STRIDE] != 0;

    for (int rr = 0; rr < MW_REQ / 4; ++rr) {
        const int r = w + 4 * rr, b = b0 + r;
        const int pb = b < n ? hdr[1 + b] : 0, pe = b < n ? hdr[2 + b] : 0;
        const bool live = b < n && pe > pb && S > 0 && planned;
        const int k_lo = live ? pb / S : 0, nk = live ? (pe - 1) / S - k_lo + 1 : 0;
        const int64_t s0 = (int64_t)(k_lo + b) * Hq + h;  // slot row of partial k: s0 + k Hq
        float M = -INFINITY;
        for (int k = lane; k < nk; k += 64) M = fmaxf(M, wm[s0 + (int64_t)k * Hq]);
        M = wave_max(M);
        const float wk = lane < nk ? exp2f(wm[s0 + (int64_t)lane * Hq] - M) : 0.f;
        float l = lane < nk ? wl[s0 + (int64_t)lane * Hq] * wk : 0.f;
        for (int k = lane + 64; k < nk; k += 64) {
            const int64_t sl = s0 + (int64_t)k * Hq;
            l += wl[sl] * exp2f(wm[sl] - M);
        }
        l = wave_sum(l);
        const float inv = live ? 1.f / l : __builtin_nanf("");
        for (int c0 = 0; c0 < v_rank; c0 += 256) {
            float a[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k = 0; k < nk; ++k) {
                const int64_t sl = s0 + (int64_t)k * Hq;
                const float wt = k < 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wk), k))
                                        : exp2f(wm[sl] - M);
                const float* row = wa + sl * v_rank;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c = c0 + lane + 64 * j;
                    if (c < v_rank) a[j] = fmaf(row[c], wt, a[j]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = c0 + lane + 64 * j;
                if (c < v_rank) s_o[r * v_rank + c] = a[j] * inv;
            }
        }
        if (lane == 0) s_live[r] = live;
    }
    __syncthreads();

    // The lift: thread (dq, cp) takes output columns 8 dq .. 8 dq + 7 over rank columns
    // c = cp (mod 16), for every request of the workgroup.
    const int dq = tid & 15, cp = tid >> 4;
    float o[MW_REQ][8];
#pragma unroll
    for (int r = 0; r < MW_REQ; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[r][e] = 0.f;
    const int64_t vh = (int64_t)h * vu_s0 + 8 * dq;
    for (int c = cp; c < v_rank; c += 16) {
        float u[8];
        load8_f(vup, vh + (int64_t)c * vu_s1, DT, u);
#pragma unroll
        for (int r = 0; r < MW_REQ; ++r) {
            const float x = s_o[r * v_rank + c];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[r][e] = fmaf(x, u[e], o[r][e]);
        }
    }
    // Sum over the wave's four sixteenths (lanes l, l ^ 16, l ^ 32, l ^ 48), then over the waves.
#pragma unroll
    for (int r = 0; r < MW_REQ; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = sum_rows(o[r][e]);
            if (lane < 16) s_red[(w * MW_REQ + r) * 128 + 8 * dq + e] = v;
        }
    __syncthreads();
    for (int i = tid; i < MW_REQ * 128; i += MW_THR) {
        const int r = i >> 7, d = i & 127, b = b0 + r;
        if (b >= n) continue;
        float v = s_red[(0 * MW_REQ + r) * 128 + d] + s_red[(1 * MW_REQ + r) * 128 + d];
        v += s_red[(2 * MW_REQ + r) * 128 + d] + s_red[(3 * MW_REQ + r) * 128 + d];
        store_f(out, (int64_t)b * o_s0 + (int64_t)h * o_s1 + d, out_dt, s_live[r] ? v : __builtin_nanf(""));
    }
}

// ---------------------------------------------------------------------------
// Host side of the P @ V pass and the merge.
// ---------------------------------------------------------------------------
namespace {

constexpr int PV_NLD = 12;  // copies per wave per page, at most (the plan keeps nch <= 96)

template <int FMT>
const void* pv_pick(int mb) {
    if (mb <= 2) return (const void*)&pv_kernel<FMT, 2, PV_NLD>;
    if (mb <= 4) return (const void*)&pv_kernel<FMT, 4, PV_NLD>;
    if (mb <= 6) return (const void*)&pv_kernel<FMT, 6, PV_NLD>;
    return (const void*)&pv_kernel<FMT, 8, PV_NLD>;
}

int raise_lds(const void* fn, int bytes) {
    static const void* raised[64];
    static int nraised = 0;
    for (int i = 0; i < nraised; ++i)
        if (raised[i] == fn) return STARKV_OK;
    SKV_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    if (nraised < 64) raised[nraised++] = fn;
    return STARKV_OK;
}

}  // namespace

// The window plan of the P @ V pass: columns per launch (a multiple of 32) and the LDS
// geometry. Table columns: bf16/fp16, the V columns; 3.2-bit, the outlier columns up to
// a multiple of 32, then the inlier columns.
struct PvPlan {
    int tcols;     // table columns in all
    int cw;        // window width (columns per launch)
    int nbuf, nch, nld, lds;
    int ng, v_off; // per-launch copy geometry (bf16/fp16: per window; 3.2-bit: all V bytes)
    bool ok;
};

static PvPlan pv_plan(int fmt, int k_width, int v_rank, int vs_off, int vq_off, int v_nout, int v_bytes) {
    PvPlan pl{};
    const int o32 = (v_nout + 31) & ~31;
    pl.tcols = fmt == FMT_Q4 ? o32 + (v_rank - v_nout) : v_rank;
    const int ncb_all = (pl.tcols + 31) / 32;
    // Candidate windows from wide to narrow; the first whose pages fit.
    for (int cbw = std::min(ncb_all, 64); cbw >= 1; --cbw) {
        const int cw = 32 * cbw;
        int ng, v_off, tab = 0;
        if (fmt == FMT_Q4) {
            v_off = vs_off & ~15;
            ng = (vq_off + v_bytes + 15) / 16 - v_off / 16;
            tab = cbw * 1024;
        } else {
            v_off = 2 * k_width;
            ng = cw / 8;
        }
        const int nch = (ng + 3) / 4 + 3;
        for (int nbuf = 3; nbuf >= 2; --nbuf) {
            const int lds = nbuf * nch * 1024 + tab + 1024;
            if (lds <= PV_MAX_DYN_LDS && (nch + NWAVE - 1) / NWAVE <= 12) {
                pl.cw = cw;
                pl.nbuf = nbuf;
                pl.nch = nch;
                pl.nld = (nch + NWAVE - 1) / NWAVE;
                pl.lds = lds;
                pl.ng = ng;
                pl.v_off = v_off;
                pl.ok = true;
                return pl;
            }
        }
    }
    pl.ok = false;
    return pl;
}

int launch_pv(const DecodeParams& p, int fmt, int grid, hipStream_t stream) {
    const int v_bytes = p.v_nbo + (p.v_rank - p.v_nout + 1) / 2;
    const PvPlan pl = pv_plan(fmt, p.k_width, p.v_rank, p.vs_off, p.vq_off, p.v_nout, v_bytes);
    SKV_CHECK(pl.ok, "decode: no P @ V window fits in LDS (v_rank %d)", p.v_rank);
    PvParams a;
    memset(&a, 0, sizeof(a));
    a.cache = p.cache; a.c_s0 = p.c_s0; a.c_s1 = (int)p.c_s1; a.bs_shift = p.bs_shift;
    a.bt = p.bt; a.bt_s0 = p.bt_s0; a.bt_s1 = p.bt_s1;
    a.n = p.n; a.Hq = p.Hq; a.v_rank = p.v_rank;
    a.ng = pl.ng;
    a.vs_rel = p.vs_off - pl.v_off;
    a.vq_rel = p.vq_off - pl.v_off;
    a.v_nout = p.v_nout; a.v_nbo = p.v_nbo; a.o32 = (p.v_nout + 31) & ~31;
    a.nch = pl.nch; a.nld = pl.nld; a.nbuf = pl.nbuf; a.buf_bytes = pl.nch * 1024;
    a.tab = pl.nbuf * pl.nch * 1024;
    a.lds_bytes = pl.lds;
    a.ws = p.ws; a.ws_plan = p.ws_plan; a.ws_m = p.ws_m; a.ws_acc = p.ws_acc; a.ws_lg = p.ws_lg; a.lcap = p.lcap;
    for (int c0 = 0; c0 < pl.tcols; c0 += pl.cw) {
        a.c0 = c0;
        a.ncb = (std::min(pl.cw, pl.tcols - c0) + 31) / 32;
        a.v_off = fmt == FMT_Q4 ? pl.v_off : pl.v_off + 2 * c0;
        const int mb = (a.ncb + NWAVE - 1) / NWAVE;
        const void* fn = fmt == FMT_BF16 ? pv_pick<FMT_BF16>(mb)
                         : fmt == FMT_F16 ? pv_pick<FMT_F16>(mb)
                                          : pv_pick<FMT_Q4>(mb);
        int rc = raise_lds(fn, PV_MAX_DYN_LDS);
        if (rc) return rc;
        void* args[] = {(void*)&a};
        SKV_HIP(hipLaunchKernel(fn, dim3(grid), dim3(NTHR), args, (size_t)a.lds_bytes, stream));
    }
    return STARKV_OK;
}

bool pv_fits(int fmt, int k_width, int v_rank, int vs_off, int vq_off, int v_nout, int v_bytes) {
    return pv_plan(fmt, k_width, v_rank, vs_off, vq_off, v_nout, v_bytes).ok;
}

int launch_merge_wide(const DecodeParams& p, int w_dt, const void* vup, int64_t vu_s0, int64_t vu_s1, void* out,
                      int64_t o_s0, int64_t o_s1, int out_dt, hipStream_t stream) {
    const size_t lds = merge_wide_lds(p.v_rank);
    SKV_CHECK(lds <= (size_t)PV_MAX_DYN_LDS, "decode: v_rank %d too large for the merge", p.v_rank);
    const dim3 grid(p.Hq, (p.n + MW_REQ - 1) / MW_REQ);
    const void* fn = w_dt == STARKV_BF16 ? (const void*)&merge_wide_kernel<STARKV_BF16>
                     : w_dt == STARKV_F16 ? (const void*)&merge_wide_kernel<STARKV_F16>
                                          : (const void*)&merge_wide_kernel<STARKV_F32>;
    int rc = raise_lds(fn, PV_MAX_DYN_LDS);
    if (rc) return rc;
    const uint8_t* ws = p.ws;
    size_t wp = p.ws_plan, wm = p.ws_m, wl = p.ws_l, wa = p.ws_acc;
    int n = p.n, Hq = p.Hq, vr = p.v_rank;
    void* args[] = {(void*)&ws, (void*)&wp, (void*)&wm, (void*)&wl, (void*)&wa, (void*)&n, (void*)&Hq, (void*)&vr,
                    (void*)&vup, (void*)&vu_s0, (void*)&vu_s1, (void*)&out, (void*)&o_s0, (void*)&o_s1,
                    (void*)&out_dt};
    SKV_HIP(hipLaunchKernel(fn, grid, dim3(MW_THR), args, lds, stream));
    return STARKV_OK;
}

}  // namespace starkv
