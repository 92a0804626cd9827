// bf16/fp16 low-rank paged decode: the decode launch of starkv_lowrank_decode
// (decode.hip holds the setup, fold and merge launches and the host entry points).
//
// One persistent workgroup of 8 waves per CU walks its contiguous range of pages (16
// tokens each), one page record per page. Each wave owns whole query heads and holds their rank tiles of AB
// (q folded into U) in VGPRs. Per page: z = AB . [cos|sin]^T on MFMA, the lanes fold z
// with the codes, the wave's heads run an online softmax, and P @ V accumulates on MFMA.
//
// LDS. The page buffers (three, or two when a page is too large to fit three times) are
// interleaved at 1 KB: chunk c of buffer b sits at byte c * NBUF KB + b KB of the dynamic
// block. Every read of the current page is a per-lane address computed once per kernel
// plus the immediate b * 1024, so the page loop does no address arithmetic. The chunks
// of a page:
//   0 .. 3            cos/sin rows 4c .. 4c+3, 256 B per row; granule g of row r is
//                     stored at granule g ^ r, so the 16 rows of an MFMA operand read
//                     hit distinct banks
//   4 .. 4+2NB-1      V codes, row t at t * NB * 128 B (columns past v_rank unused)
//   4+2NB+m           K codes of code tiles 2m (at +0) and 2m+1 (at +512), row r at +32 r
//   nch .. nch+2NB-1  (not copied) the page's V transposed into the P @ V B operand:
//                     entry (step s, column L) is 4 tokens x 16 bit at byte (s 64 NB + L) 8
// After the barrier of page j every thread moves two V codes of one token into that
// table, and page j's P @ V runs one page later, one 4-token step per K tile, so its
// reads and MFMAs ride under the next page's K side (the table survives the copies that
// refill the page's buffer).
// Copy i of wave w moves chunk 8 i + w; lane q's offset inside the page depends only on
// (chunk, q) and is computed once (`doff`). Copies past the page's chunks land in a
// 1 KB dummy block after the buffers and read nothing.
//
// NB = 0 is the logits pass of a two-pass call (V ranks too wide for P @ V in this
// kernel): no V chunks, no V table and no P @ V; the softmax stores each valid logit
// (log2 domain, fp32) into the workspace logits buffer and keeps m and l for the
// split-K partials, and decode_wide.hip's pass runs P @ V from those logits.

#include "decode_pages.hpp"

namespace starkv {

namespace {

// Dynamic LDS limit: 160 KB per CU minus the kernel's static arrays (partial logits,
// P, alpha, head ids: under 12 KB).
constexpr int LR_MAX_DYN_LDS = 160 * 1024 - 12 * 1024;

template <int NB>
struct LrChunks {
    static constexpr int V0 = CS_CHUNKS;           // first V chunk
    static constexpr int K0 = CS_CHUNKS + 2 * NB;  // first K chunk
    static constexpr int VPITCH = NB * 128;        // V row pitch in LDS
};

// Per-lane LDS byte addresses (buffer 0), fixed for the whole kernel.
template <int MTV, int NB>
struct LaneAddr {
    uint32_t cs[4];               // B operand: row lr, granule 4 ks + lg
    uint32_t k[MTV];              // slot i: 8 code bytes of row lr, ranks 4 lg .. 4 lg + 3
    uint32_t vt;                  // V table entry (0, lane)
    uint32_t cv_rd[NB > 0 ? NB : 1], cv_wr[NB > 0 ? NB : 1];  // V transpose: the two codes read, the entry written
    int lg;                       // NB = 0: this lane's logit offset in a page's block (q head x 16 + token)
    uint32_t st[(MTV + 3) / 4];   // partial-logit row of this lane's slot in each group of 4
    uint32_t sm;                  // softmax: first of the 4 rows of head lane >> 4
    uint32_t pw, pr;              // P: write (head lane >> 4, token lane & 15), read (head lane & 3)
    uint32_t base;                // the page buffers (wave-uniform)
};

// Copy points of an iteration: 0 right after the barrier, 1 .. MTV after each K tile
// (which also carry the previous page's P @ V), MTV + 1 after the softmax.
template <int MTV>
struct LrSched {
    static constexpr int NPOS = MTV + 2;
    static constexpr float time(int pos) {
        return pos == 0 ? 0.f : pos <= MTV ? 0.75f * (float)pos / (float)MTV : 0.9f;
    }
};

// Byte offset of V-table entry (step s, column L) from the table's first chunk.
template <int NBUF>
__device__ __forceinline__ uint32_t vt_offset(int logical) {
    return (uint32_t)((logical >> 10) * page_stride<NBUF>() + (logical & 1023));
}
template <int NB, int NBUF>
constexpr uint32_t vt_step_offset(int s, int nb) {  // entry (s, 64 nb) for lane 0
    return (uint32_t)(((s * NB + nb) >> 1) * page_stride<NBUF>() + ((s * NB + nb) & 1) * 512);
}

// z . codes for one tile: this lane's 4 z values (rows 4 lg .. 4 lg + 3) times its 4
// codes (8 bytes).
template <int FMT>
__device__ __forceinline__ float tile_dot(const f32x4_t& z, uint2 w) {
    if (FMT == FMT_BF16) {
        float v = __uint_as_float(w.x << 16) * z[0];
        v = fmaf(__uint_as_float(w.x & 0xffff0000u), z[1], v);
        v = fmaf(__uint_as_float(w.y << 16), z[2], v);
        return fmaf(__uint_as_float(w.y & 0xffff0000u), z[3], v);
    } else {
        return dot2(as_h2(w.x), cvt_h2(z[0], z[1]), dot2(as_h2(w.y), cvt_h2(z[2], z[3]), 0.f));
    }
}

// K side of one page (buffer B): MTV slots from VGPR AB, more from L2. Each group of
// 4 slots is summed over the row groups with the lane swaps and stored as 4 rows.
// `hook(i)` runs after tile i's lane work (i a constant once the loop is unrolled).
template <int FMT, int MTV, int NB, int B, int NLD, int BN, int NBUF, class Hook>
__device__ __forceinline__ void k_side(const DecodeParams& p, const LaneAddr<MTV, NB>& la, const half8_t (&ab)[MTV][4],
                                       int ntw, int nh, bool fast, uint32_t sp, int lane, int wave, int cur_b,
                                       const DmaConst& dc, const DmaPage& dp, const uint32_t (&doff)[NLD],
                                       Hook&& hook) {
    half8_t csb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) csb[ks] = lds_ld<half8_t>(la.cs[ks] + B * 1024);
    float v[4];
#pragma unroll
    for (int i = 0; i < MTV; ++i) {
        const f32x4_t z = mfma_tile(ab[i], csb);
        v[i & 3] = tile_dot<FMT>(z, lds_ld2(la.k[i] + B * 1024));
        hook(i);
        if ((i & 3) == 3 || i == MTV - 1) {
            const float r = sum_rows4(v[0], (i & 3) >= 1 ? v[1] : 0.f, (i & 3) >= 2 ? v[2] : 0.f,
                                      (i & 3) >= 3 ? v[3] : 0.f);
            lds_st<float>(la.st[i >> 2], r);
        }
        copies_at<LrSched<MTV>, NLD, BN, NBUF>(1 + i, dc, dp, opaque_s(wave), doff);
    }
    if (ntw > MTV) {  // slots past MTV: AB from the workspace (L2) on every page
        const int lg = lane >> 4, lr = lane & 15;
        cint_p pw = (cint_p)(p.ws + p.ws_plan) + wave * PLAN_STRIDE;
        const half8_t* abg = (const half8_t*)(p.ws + p.ws_ab + (size_t)cur_b * p.TT * AB_TILE_BYTES);
        for (int i = MTV; i < ntw; ++i) {
            const uint32_t wd = (uint32_t)pw[PW_SLOTS + i];
            const int t = sw_tile(wd);
            half8_t a[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) a[ks] = abg[(t * 4 + ks) * 64 + lane];
            const int T = sw_code(wd);
            const uint32_t ka = la.base + (uint32_t)((LrChunks<NB>::K0 + (T >> 1)) * page_stride<NBUF>() + (T & 1) * 512 +
                                                        lr * 32 + 8 * lg + B * 1024);
            const float r = sum_rows(tile_dot<FMT>(mfma_tile(a, csb), lds_ld2(ka)));
            if (lane < 16) lds_st<float>(sp + (uint32_t)(sw_row(wd) * TILE_TOK + lr) * 4, r);
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): no tracked load left pending
    }
}

// Online softmax of the wave's heads (head lane >> 4 on a 16-lane row, token lane & 15).
// Returns true when some head's reference max moved (acc needs rescaling by alpha).
// LG (the logits pass): no P; each valid logit goes to lgd instead.
template <int FMT, bool LG = false>
__device__ __forceinline__ bool softmax_page(SmState& sm, const uint32_t sm_addr, bool fast, uint32_t sp, int nh,
                                             uint32_t pw_addr, uint32_t plo_off, uint32_t salpha, uint32_t shfn, int lane, int tok0,
                                             int lo, int hi, float* lgd = nullptr) {
    const int kh = lane >> 4, lr = lane & 15;
    float s;
    if (fast) {
        s = (lds_ld<float>(sm_addr) + lds_ld<float>(sm_addr + 64)) +
            (lds_ld<float>(sm_addr + 128) + lds_ld<float>(sm_addr + 192));
    } else {
        s = 0.f;
        const int hfn = head_slots(shfn, lane);
        for (int t = 0; t < (hfn >> 8); ++t) s += lds_ld<float>(sp + (uint32_t)(((hfn & 255) + t) * TILE_TOK + lr) * 4);
    }
    const int tok = tok0 + lr;
    const bool valid = tok >= lo && tok < hi && kh < nh;
    s = valid ? s : -INFINITY;
    if (LG && valid) *lgd = s;
    float alpha = 1.f;
    bool moved = false;
    if (__builtin_amdgcn_ballot_w64(s > sm.m + LAZY_MAX) != 0) {
        const float mn = fmaxf(sm.m, row16_max(s));
        alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(sm.m - mn);
        sm.m = mn;
        moved = true;
        if (!LG && lr == 0) lds_st<float>(salpha + 4 * (opaque(lane) >> 4), alpha);
    }
    const float pe = s == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - sm.m);
    sm.l = fmaf(sm.l, alpha, pe);
    if (LG) return moved;
    if (FMT == FMT_BF16) {
        // P = hi + lo in two bfloat16 parts: the P @ V product keeps ~16 bits of P.
        const __bf16 ph = (__bf16)pe;
        const __bf16 pl = (__bf16)(pe - (float)ph);
        lds_st<uint16_t>(pw_addr, __builtin_bit_cast(uint16_t, ph));
        lds_st<uint16_t>(pw_addr + plo_off, __builtin_bit_cast(uint16_t, pl));
    } else {
        lds_st<uint16_t>(pw_addr, __builtin_bit_cast(uint16_t, (_Float16)pe));
    }
    return moved;
}

// Moves this thread's two V codes of one token (the word xv[k], columns 2 c, 2 c + 1)
// into the V table of buffer B.
template <int NB, int B>
__device__ __forceinline__ void lr_transpose_v(const uint32_t (&xv)[NB], const uint32_t (&wr)[NB]) {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        lds_st<uint16_t>(wr[k] + B * 1024, (uint16_t)xv[k]);
        lds_st<uint16_t>(wr[k] + B * 1024 + 8, (uint16_t)(xv[k] >> 16));
    }
}

// One 4-token step of acc[nb] += P[4 heads, 16 tokens] @ V[16 tokens, 64 columns] on
// v_mfma_f32_4x4x4_16b with block 0's A broadcast (cbsz 4): lanes 0..3 hold P[head l]
// [4 tokens] (bf16: a high and a low part), lane l holds V[4 tokens][column 64 nb + l],
// and the result lands in lane l as acc[nb][head] for its column. The operands are read
// one K tile before the MFMAs that use them.
template <int NB>
struct PvStep {
    uint2 ph, pl, b[NB > 0 ? NB : 1];
};
template <int FMT, int NB, int B, int NBUF>
__device__ __forceinline__ void pv_load(PvStep<NB>& q, uint32_t pr, uint32_t plo_off, uint32_t vt, int s) {
    q.ph = lds_ld2(pr + 8 * s);
    if (FMT == FMT_BF16) q.pl = lds_ld2(pr + plo_off + 8 * s);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) q.b[nb] = lds_ld2(vt + vt_step_offset<NB, NBUF>(s, nb) + B * 1024);
}
template <int FMT, int NB>
__device__ __forceinline__ void pv_mfma(f32x4_t (&acc)[NB > 0 ? NB : 1], const PvStep<NB>& q) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (FMT == FMT_BF16) {
            acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(short4_t, q.ph),
                                                             __builtin_bit_cast(short4_t, q.b[nb]), acc[nb], 4, 0, 0);
            acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(short4_t, q.pl),
                                                             __builtin_bit_cast(short4_t, q.b[nb]), acc[nb], 4, 0, 0);
        } else {
            acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, q.ph),
                                                         __builtin_bit_cast(half4_t, q.b[nb]), acc[nb], 4, 0, 0);
        }
    }
}

// The whole P @ V of the page whose V table is in buffer B (the last page, after the loop).
template <int FMT, int NB, int NBUF>
__device__ __forceinline__ void pv_page(f32x4_t (&acc)[NB > 0 ? NB : 1], uint32_t pr, uint32_t plo_off, uint32_t vt,
                                        uint32_t salpha, bool rescale) {
    if (rescale) {
        const f32x4_t al = lds_ld<f32x4_t>(salpha);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[nb][e] *= al[e];
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        PvStep<NB> q;
        pv_load<FMT, NB, 0, NBUF>(q, pr, plo_off, vt, s);
        pv_mfma<FMT, NB>(acc, q);
    }
}

struct LrLoop : PageLoop {
    bool pv_moved;  // the previous page's softmax moved a reference max
    bool pv_end;    // the previous page ended its request: flush after its P @ V
    int pv_b;       // its request
    int pv_buf;     // its buffer, when the loop ends
};

// One page of the loop: buffer BC holds page j (copied NBUF - 1 pages ago); buffer BN
// receives page j + NBUF - 1 (its previous content, page j - 1, is done on every wave
// once the barrier is passed, except page j - 1's V table, which this iteration's P @ V
// reads and the copies do not touch).
template <int FMT, int MTV, int NB, int NLD, int BC, int BN, int NBUF>
__device__ __forceinline__ bool lr_iter(LrLoop& st, const DmaConst& dc, const LaneAddr<MTV, NB>& la,
                                        half8_t (&ab)[MTV][4], f32x4_t (&acc)[NB > 0 ? NB : 1], SmState& sm,
                                        const uint32_t (&doff)[NLD], int ntw, int nh, bool fast, uint32_t sp,
                                        uint32_t plo_off, uint32_t salpha, uint32_t shfn, const int* sqh, int lane, int wave) {
    const DecodeParams& p = params();
    if (st.j >= st.end) {
        st.pv_buf = BN;  // the last page's buffer: its P @ V runs after the loop
        return false;
    }
    const int b = pr_b(st.rc.bits), k = st.rc.k, rows = pr_rows(st.rc.bits);
    if (page_starts_seg(st)) {
        // This request's AB into registers; slots past the wave's tiles load tile 0.
        cint_p pw = (cint_p)(p.ws + p.ws_plan) + wave * PLAN_STRIDE;
        const half8_t* abp = (const half8_t*)(p.ws + p.ws_ab + (size_t)b * p.TT * AB_TILE_BYTES);
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            const int t = pw[8 + i];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ab[i][ks] = abp[(t * 4 + ks) * 64 + lane];
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    }
    SKV_WAIT_VM_LGKM0(NBUF == 3 ? NLD : 0);  // only the copies of page j + 1 may still be in flight
    lds_barrier();  // page j is in LDS, page j - 1's V table is complete; every wave is done with page j - 1
    const int jl = st.j + NBUF - 1;  // the page whose copies issue now
    const DmaPage dp = dma_setup(dc, NBUF == 3 ? st.r2 : st.r1, jl < st.end);
    // The record of the page the next iteration copies: it arrives under the next wait.
    const PageRec next = jl + 1 < st.end ? page_rec(p, jl + 1) : st.rc;
    // Page j's V codes for the transpose, read first; page j - 1's P @ V (its P was 0
    // before the first page) runs inside the K side: its rescale first, then one step
    // per tile.
    uint32_t xv[NB > 0 ? NB : 1];
#pragma unroll
    for (int q = 0; q < NB; ++q) xv[q] = lds_ld<uint32_t>(la.cv_rd[q] + BC * 1024);
    if (NB > 0 && st.pv_moved) {
        const f32x4_t al = lds_ld<f32x4_t>(salpha);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[nb][e] *= al[e];
    }
    copies_at<LrSched<MTV>, NLD, BN, NBUF>(0, dc, dp, opaque_s(wave), doff);
    PvStep<NB> pq;
    auto hook = [&](int i) {
        if constexpr (NB > 0) {
            if (i == 0) lr_transpose_v<NB, BC>(xv, la.cv_wr);
            if (i >= 1 && i <= 4) pv_mfma<FMT, NB>(acc, pq);
            if (i <= 3) pv_load<FMT, NB, BN, NBUF>(pq, la.pr, plo_off, la.vt, i);
        }
    };
    k_side<FMT, MTV, NB, BC, NLD, BN, NBUF>(p, la, ab, ntw, nh, fast, sp, lane, wave, b, dc, dp, doff, hook);
#pragma unroll
    for (int i = MTV; i <= 4; ++i) hook(i);  // the P @ V steps a short K side left
    if constexpr (NB > 0) {
        if (st.pv_end) flush_partial<NB>(p, sm, acc, nh, st.pv_b + st.g, sqh, lane);
        st.pv_moved = softmax_page<FMT>(sm, la.sm, fast, sp, nh, la.pw, plo_off, salpha, shfn, lane, 0, 0, rows);
    } else {
        // The logits pass: page j's logits into the request's rows, and its partial
        // (m, l) flushed right away when page j ends the request.
        float* lgd = (float*)(p.ws + p.ws_lg) + ((int64_t)b * (p.lcap / TILE_TOK) + k) * p.Hq * TILE_TOK + la.lg;
        softmax_page<FMT, true>(sm, la.sm, fast, sp, nh, la.pw, plo_off, salpha, shfn, lane, 0, 0, rows, lgd);
    }
    copies_at<LrSched<MTV>, NLD, BN, NBUF>(MTV + 1, dc, dp, opaque_s(wave), doff);
    const bool seg_end = page_ends_seg(st);
    if constexpr (NB == 0) {
        if (seg_end) flush_partial<0>(p, sm, acc, nh, b + st.g, sqh, lane);
    }
    st.pv_end = seg_end;
    st.pv_b = b;
    page_loop_next<NBUF>(st, next);
    return true;
}

template <int FMT, int MTV, int NB, int NLD, int NBUF>
__global__ __launch_bounds__(NTHR) void lowrank_kernel(const DecodeParams p0) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_pages[];
    __shared__ __attribute__((aligned(16))) float s_part[NWAVE][(MAX_SLOTS + 1) * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_p[NWAVE][4 * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_plo[FMT == FMT_BF16 ? NWAVE : 1][4 * TILE_TOK];
    __shared__ __attribute__((aligned(16))) float s_alpha[NWAVE][4];
    __shared__ int s_qh[NWAVE][4];
    __shared__ int s_hfn[NWAVE][4];  // per local head: first slot | slots << 8
    typedef LrChunks<NB> C;

    const DecodeParams& p = params();
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    const int lg = lane >> 4, lr = lane & 15;
    cint_p plan = (cint_p)(p.ws + p.ws_plan);
    // Page buffers and partial-logit rows start zeroed: rows past a request's end are
    // never copied and must hold finite values (P is 0 there); a head's partial rows
    // past its slots are summed as zeros. Done first: it overlaps the header loads.
    for (int i = tid; i < p.lds_bytes / 16; i += NTHR) ((uint4*)s_pages)[i] = make_uint4(0, 0, 0, 0);
    for (int i = tid; i < NWAVE * (MAX_SLOTS + 1) * TILE_TOK; i += NTHR) (&s_part[0][0])[i] = 0.f;
    if (tid < NWAVE * 4) (&s_alpha[0][0])[tid] = 1.f;
    for (int i = tid; i < NWAVE * 4 * TILE_TOK; i += NTHR) {  // P before the first page
        (&s_p[0][0])[i] = 0;
        if (FMT == FMT_BF16) (&s_plo[0][0])[i] = 0;
    }
    const int planned = plan[NWAVE * PLAN_STRIDE], hS = ((cint_p)p.ws)[0], htot = ((cint_p)p.ws)[1 + p.n];
    __syncthreads();  // the zero fill is done on every wave before a page copy lands
    if (planned == 0) return;  // no wave plan: the merge reports NaN
    LrLoop st;
    if (!page_loop_init<NBUF>(st, p, xcd_range(blockIdx.x, gridDim.x), hS, htot)) return;
    // The first pages' copies go out as soon as their records are in: the rest of the
    // setup (the wave plan, the lane addresses) runs under their latency.
    const uint32_t base = lds_addr(s_pages);
    uint32_t doff[NLD];  // copy offsets of this lane inside a page, per copy i (chunk 8 i + wave)
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        uint32_t off = 0x80000000u;  // past the descriptor range: no memory access
        if (ch < CS_CHUNKS) {
            off = cs_copy_offset(ch, lane, p.cs_s0b);
        } else if (ch < C::K0) {
            if constexpr (NB > 0) {
                const int vb = (ch - C::V0) * 1024 + 16 * lane;  // byte inside the V rows
                const int row = vb / C::VPITCH, col = vb % C::VPITCH;
                if (col < 2 * p.v_rank) off = (uint32_t)(row * (int)p.c_s1 + 2 * p.v_col + col);
            }
        } else if (ch < p.nch) {
            const int Tc = 2 * (ch - C::K0) + (lane >> 5), r = (lane >> 1) & 15, h = lane & 1;
            if (Tc < p.k_width / 16) off = (uint32_t)(r * (int)p.c_s1 + 32 * Tc + 16 * h);
        }
        doff[i] = off;
    }
    const DmaConst dc = dma_const<NBUF>(p, base, wave, base + (uint32_t)((p.nch + 2 * NB) * page_stride<NBUF>()));
    dma_page<NLD, 0, NBUF>(dc, st.rc, true, wave, doff);
    if (NBUF == 3) dma_page<NLD, 1, NBUF>(dc, st.r1, st.beg + 1 < st.end, wave, doff);

    // This wave's plan: slots (rank tiles) and heads (at most 4: Hq <= 32).
    cint_p pw = plan + wave * PLAN_STRIDE;
    const int ntw = pw[0], nh = pw[1];
    const bool fast = pw[3] != 0;
    const uint32_t sp = lds_addr(&s_part[wave][0]);
    LaneAddr<MTV, NB> la;
    uint32_t swd[MTV];  // the wave's slot words (plan order), read with a few wide scalar loads
#pragma unroll
    for (int i = 0; i < MTV; ++i) swd[i] = (uint32_t)pw[PW_SLOTS + i];
    {
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            const int Tc = sw_code(swd[i]);  // code tile: first cache lane / 16
            la.k[i] = vgpr_pin(base + (uint32_t)((C::K0 + (Tc >> 1)) * page_stride<NBUF>() + (Tc & 1) * 512 +
                                                 lr * 32 + 8 * lg));
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            la.cs[ks] = base + cs_read_offset<NBUF>(ks, lg, lr);
        la.base = base;
        const uint32_t vt0 = base + (uint32_t)(p.nch * page_stride<NBUF>());  // V table
        la.vt = vt0 + 8 * lane;
        // V transpose: token t = tid % 16, columns L, L + 1 with L = 2 (tid / 16) + 64 k.
        const int t = tid & 15;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int L = 2 * (tid >> 4) + 64 * k;
            const int vb = t * C::VPITCH + 2 * L;  // byte inside the V rows
            la.cv_rd[k] = base + (uint32_t)((C::V0 + (vb >> 10)) * page_stride<NBUF>() + (vb & 1023));
            la.cv_wr[k] = vt0 + vt_offset<NBUF>((((t >> 2) * 64 * NB + L) << 3) + (t & 3) * 2);
        }
        la.lg = (lg < nh ? pw[32 + lg] : 0) * TILE_TOK + lr;
        const int rslot = ((lg & 1) << 1) | (lg >> 1);  // sum_rows4 puts inputs (a, b, c, d) in rows (0, 2, 1, 3)
#pragma unroll
        for (int g = 0; g < (MTV + 3) / 4; ++g) {
            int row = MAX_SLOTS;  // the row of slot 4 g + rslot (past MTV: the spare row)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * g + j < MTV && rslot == j) row = sw_row(swd[4 * g + j < MTV ? 4 * g + j : 0]);
            la.st[g] = sp + (uint32_t)(row * TILE_TOK + lr) * 4;
        }
        la.sm = sp + (uint32_t)(4 * lg * TILE_TOK + lr) * 4;
        la.pw = lds_addr(&s_p[wave][0]) + (uint32_t)(lg * TILE_TOK + lr) * 2;
        la.pr = lds_addr(&s_p[wave][0]) + (uint32_t)(lane & 3) * TILE_TOK * 2;
        // Whole-VGPR lane addresses (see vgpr_pin).
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) la.cs[ks] = vgpr_pin(la.cs[ks]);
#pragma unroll
        for (int g = 0; g < (MTV + 3) / 4; ++g) la.st[g] = vgpr_pin(la.st[g]);
        la.sm = vgpr_pin(la.sm);
        la.pw = vgpr_pin(la.pw);
        la.pr = vgpr_pin(la.pr);
        la.vt = vgpr_pin(la.vt);
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            la.cv_rd[k] = vgpr_pin(la.cv_rd[k]);
            la.cv_wr[k] = vgpr_pin(la.cv_wr[k]);
        }
    }
    const uint32_t plo_off = lds_addr(&s_plo[FMT == FMT_BF16 ? wave : 0][0]) - lds_addr(&s_p[wave][0]);
    const uint32_t salpha = lds_addr(&s_alpha[wave][0]);
    if (lane < 4) s_qh[wave][lane] = lane < nh ? pw[32 + lane] : 0;
    SmState sm;
    if (lane < 4) s_hfn[wave][lane] = lane < nh ? pw[40 + lane] | (pw[48 + lane] << 8) : 0;
    const uint32_t shfn = lds_addr(&s_hfn[wave][0]);
    sm.m = -INFINITY;
    sm.l = 0.f;

    __syncthreads();

    st.pv_moved = false;
    st.pv_end = false;
    st.pv_b = 0;
    st.pv_buf = 0;

    half8_t ab[MTV][4];
    f32x4_t acc[NB > 0 ? NB : 1];
#pragma unroll
    for (int k = 0; k < (NB > 0 ? NB : 1); ++k) acc[k] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    const int* sqh = &s_qh[wave][0];
    if (NBUF == 3) {
        while (true) {
            if (!lr_iter<FMT, MTV, NB, NLD, 0, 2, NBUF>(st, dc, la, ab, acc, sm, doff, ntw, nh, fast, sp, plo_off, salpha, shfn, sqh,
                                                  lane, wave))
                break;
            if (!lr_iter<FMT, MTV, NB, NLD, 1, 0, NBUF>(st, dc, la, ab, acc, sm, doff, ntw, nh, fast, sp, plo_off, salpha, shfn, sqh,
                                                  lane, wave))
                break;
            if (!lr_iter<FMT, MTV, NB, NLD, 2, 1, NBUF>(st, dc, la, ab, acc, sm, doff, ntw, nh, fast, sp, plo_off, salpha, shfn, sqh,
                                                  lane, wave))
                break;
        }
    } else {  // two buffers: page j + 1 goes into the buffer page j - 1 left
        while (true) {
            if (!lr_iter<FMT, MTV, NB, NLD, 0, 1, NBUF>(st, dc, la, ab, acc, sm, doff, ntw, nh, fast, sp, plo_off, salpha,
                                                       shfn, sqh, lane, wave))
                break;
            if (!lr_iter<FMT, MTV, NB, NLD, 1, 0, NBUF>(st, dc, la, ab, acc, sm, doff, ntw, nh, fast, sp, plo_off, salpha,
                                                       shfn, sqh, lane, wave))
                break;
        }
    }
    // The last page's P @ V, once its V table is visible to every wave.
    SKV_WAIT_VM_LGKM0(0);  // also: no copy may land after the workgroup ends
    if constexpr (NB > 0) {
        lds_barrier();
        pv_page<FMT, NB, NBUF>(acc, la.pr, plo_off, la.vt + (uint32_t)st.pv_buf * 1024u, salpha, st.pv_moved);
        flush_partial<NB>(p, sm, acc, nh, st.pv_b + st.g, sqh, lane);
    }
}

// The instantiations that run without scratch spills: MTV tiles per wave held in VGPRs
// with NB V blocks. Only these are compiled (lowrank_mtv picks among them).
constexpr bool lr_spill_free(int mtv, int nb) { return mtv <= 8 || (mtv == 9 && nb <= 2) || (mtv == 10 && nb <= 1); }

template <int FMT, int MTV, int NB, int NLD, int NBUF>
const void* inst() {
    if constexpr (lr_spill_free(MTV, NB)) return (const void*)&lowrank_kernel<FMT, MTV, NB, NLD, NBUF>;
    return nullptr;
}

template <int FMT, int MTV, int NLD, int NBUF>
const void* pick_nb(int nb) {
    if (nb <= 0) return inst<FMT, MTV, 0, NLD, NBUF>();
    if (nb <= 1) return inst<FMT, MTV, 1, NLD, NBUF>();
    if (nb <= 2) return inst<FMT, MTV, 2, NLD, NBUF>();
    return inst<FMT, MTV, 4, NLD, NBUF>();
}

template <int FMT, int NLD, int NBUF>
const void* pick_mtv(int mtv, int nb) {
    return mtv == 4 ? pick_nb<FMT, 4, NLD, NBUF>(nb)
           : mtv == 8 ? pick_nb<FMT, 8, NLD, NBUF>(nb)
           : mtv == 9 ? pick_nb<FMT, 9, NLD, NBUF>(nb)
                      : pick_nb<FMT, 10, NLD, NBUF>(nb);
}

template <int FMT>
const void* pick(int nbuf, int nld, int mtv, int nb) {
    if (nbuf == 2) return pick_mtv<FMT, 8, 2>(mtv, nb);
    return nld <= 3 ? pick_mtv<FMT, 3, 3>(mtv, nb) : pick_mtv<FMT, 6, 3>(mtv, nb);
}

int nb_blocks(int nb) { return nb <= 0 ? 0 : nb <= 1 ? 1 : nb <= 2 ? 2 : 4; }

}  // namespace

int lowrank_chunks(int k_width, int nb) {
    const int tiles = k_width / 16;
    return CS_CHUNKS + 2 * nb_blocks(nb) + (tiles + 1) / 2;
}

// Page buffers: three while a page's copied chunks and its V table fit three times (48
// chunks), else two (up to 64 copied chunks); 0 if a page does not fit.
int lowrank_buffers(int k_width, int nb) {
    const int ch = lowrank_chunks(k_width, nb), all = ch + 2 * nb_blocks(nb);
    return all <= 48 && ch <= 6 * NWAVE ? 3 : ch <= 8 * NWAVE && all <= 72 ? 2 : 0;
}

// Copies per wave per page (the instantiated counts: 3 or 6 with three buffers, 8 with
// two), 0 if a page does not fit.
int lowrank_copies(int k_width, int nb) {
    const int nld = (lowrank_chunks(k_width, nb) + NWAVE - 1) / NWAVE;
    const int nbuf = lowrank_buffers(k_width, nb);
    return nbuf == 3 ? (nld <= 3 ? 3 : 6) : nbuf == 2 ? 8 : 0;
}

int lowrank_lds_bytes(int k_width, int nb) {
    return (lowrank_chunks(k_width, nb) + 2 * nb_blocks(nb)) * lowrank_buffers(k_width, nb) * 1024 + 1024;
}

// Rank tiles per wave held in VGPRs for a layer of TT rank tiles and nb V blocks (the
// one-pass kernel; nb = 0 the logits pass). The wave plan balances whole heads to within a
// tile of TT / 8, so need = ceil(TT / 8) covers every wave for the usual rank mixes (a wave
// with more streams the rest of its tiles from L2 on every page). The smallest compiled
// size >= need, or, where that one would spill with nb V blocks, the next smaller one if
// it still holds need - 1; 0 if neither runs without spills (the layer then takes the
// two-pass form, whose logits pass has none: nb = 0 never returns 0).
int lowrank_mtv(int TT, int nb) {
    static const int sizes[4] = {4, 8, 9, 10};
    const int need = (TT + NWAVE - 1) / NWAVE;
    int i = 0;
    while (i < 3 && sizes[i] < need) ++i;
    const int nbv = nb_blocks(nb);
    if (lr_spill_free(sizes[i], nbv)) return sizes[i];
    if (i > 0 && sizes[i - 1] >= need - 1 && lr_spill_free(sizes[i - 1], nbv)) return sizes[i - 1];
    return 0;
}

int launch_lowrank(const DecodeParams& p, int fmt, int nb, int grid, hipStream_t stream) {
    const int mtv = lowrank_mtv(p.TT, nb);
    const int nld = lowrank_copies(p.k_width, nb), nbuf = lowrank_buffers(p.k_width, nb);
    SKV_CHECK(mtv > 0, "decode: no spill-free kernel for %d rank tiles and %d V blocks", p.TT, nb);
    const void* fn = fmt == FMT_BF16 ? pick<FMT_BF16>(nbuf, nld, mtv, nb) : pick<FMT_F16>(nbuf, nld, mtv, nb);
    SKV_CHECK(fn != nullptr, "decode: no kernel for %d rank tiles and %d V blocks", p.TT, nb);
    static const void* raised[256];  // kernels whose dynamic-LDS limit was raised (host-side bookkeeping)
    static int nraised = 0;
    bool seen = false;
    for (int i = 0; i < nraised; ++i) seen = seen || raised[i] == fn;
    if (!seen) {
        SKV_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LR_MAX_DYN_LDS));
        if (nraised < 256) raised[nraised++] = fn;
    }
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(grid), dim3(NTHR), args, (size_t)p.lds_bytes, stream));
    return STARKV_OK;
}

}  // namespace starkv
