// Page machinery shared by the two decode kernels (decode_lowrank.hip for bf16/fp16
// codes, decode_quant.hip for 3.2-bit codes): LDS access helpers, the global->LDS page
// copies and their schedule over an iteration, and the page-loop state.
//
// Page buffers. A workgroup keeps NBUF page buffers (three: pages j, j + 1, j + 2 in
// flight; two for pages too large to fit three times) interleaved at 1 KB: chunk c of
// buffer b sits at byte c * NBUF KB + b KB of the dynamic LDS block, so a read of the
// current page is a per-lane address fixed for the whole kernel plus the immediate
// b * 1024. Chunks 0 .. 3 of a page hold its 16
// cos/sin rows (256 B per row; granule g of row r is stored at granule g ^ r, so the 16
// rows of an MFMA operand read hit distinct banks); the chunks after them are the
// kernel's own. Copy i of wave w moves chunk 8 i + w; a lane's source offset inside the
// page depends only on (chunk, lane) and is computed once. Copies past a page's chunks
// land in a 1 KB dummy block and read nothing, so every wave issues the same number of
// copies per page and the waits stay static.
#pragma once

#include "decode_common.hpp"

namespace starkv {

// Bytes between chunks c and c + 1 of one buffer.
template <int NBUF>
constexpr int page_stride() {
    return NBUF * 1024;
}
constexpr int PAGE_STRIDE = page_stride<3>();  // the three-buffer layout

typedef short short2_t __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t a) {
    return *(const __attribute__((address_space(3))) T*)(a);
}
template <typename T>
__device__ __forceinline__ void lds_st(uint32_t a, T v) {
    *(__attribute__((address_space(3))) T*)(a) = v;
}
__device__ __forceinline__ uint2 lds_ld2(uint32_t a) {
    const uint64_t v = lds_ld<uint64_t>(a);
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// A 16-byte-per-lane copy to LDS address m0 (a wave-uniform SGPR value).
__device__ __forceinline__ void copy16(const int4v_t& rsrc, uint32_t m0, uint32_t voff) { lds_copy16(rsrc, m0, voff); }

// Source offset of lane `lane`'s 16 bytes of cos/sin chunk ch (< CS_CHUNKS): row
// 4 ch + lane / 16, LDS granule g = lane % 16 holding granule g ^ row.
__device__ __forceinline__ uint32_t cs_copy_offset(int ch, int lane, int cs_s0b) {
    const int row = 4 * ch + (lane >> 4), g = lane & 15;
    return (uint32_t)(row * cs_s0b + ((g ^ row) << 4));
}

// LDS address (buffer 0, relative to the page block) of granule 4 ks + lg of cos/sin
// row lr: the B operand of v_mfma_f32_16x16x32_f16 for K-step ks.
template <int NBUF = 3>
__device__ __forceinline__ uint32_t cs_read_offset(int ks, int lg, int lr) {
    return (uint32_t)((lr >> 2) * page_stride<NBUF>() + (lr & 3) * 256 + (((4 * ks + lg) ^ lr) << 4));
}

// Loop-invariant operands of the page copies, read once from the parameter block and
// held in SGPRs.
struct DmaConst {
    int c_s1;
    const uint8_t* cs; int cs_s0b;
    int nch;
    uint32_t m0w, m0dummy;  // LDS address of this wave's first chunk (buffer 0); the dummy block
};

template <int NBUF = 3>
__device__ __forceinline__ DmaConst dma_const(const DecodeParams& p, uint32_t base, int wave, uint32_t dummy) {
    DmaConst dc;
    dc.c_s1 = (int)p.c_s1;
    dc.cs = p.cs; dc.cs_s0b = p.cs_s0b;
    dc.nch = p.nch;
    dc.m0w = base + (uint32_t)(wave * page_stride<NBUF>());
    dc.m0dummy = dummy;
    return dc;
}

// The page records, read with scalar loads (wave-uniform index): one s_load_dwordx4.
typedef const __attribute__((address_space(4))) int4v_t* crec_p;
__device__ __forceinline__ PageRec rec_of(int4v_t v) {
    PageRec r;
    r.addr = (uint64_t)(uint32_t)v[0] | ((uint64_t)(uint32_t)v[1] << 32);
    r.k = v[2];
    r.bits = (uint32_t)v[3];
    return r;
}
__device__ __forceinline__ PageRec page_rec(const DecodeParams& p, int j) {
    return rec_of(((crec_p)(p.ws + p.ws_pages))[j]);
}

// Buffer descriptors of one page: its rows and its cos/sin rows, bounded to the rows
// the request has (rows past its end are not read). Past the end of the workgroup's
// range (valid false) both are empty: the copies still issue.
struct DmaPage {
    int4v_t rkv, rcs;
};

__device__ __forceinline__ DmaPage dma_setup(const DmaConst& dc, const PageRec& r, bool valid) {
    const int rows = valid ? pr_rows(r.bits) : 0;
    DmaPage d;
    d.rkv = buffer_rsrc((const void*)(uintptr_t)r.addr, rows * dc.c_s1);
    d.rcs = buffer_rsrc(dc.cs + (int64_t)(valid ? r.k : 0) * (TILE_TOK * dc.cs_s0b), rows * dc.cs_s0b);
    return d;
}

// Copy i of this wave into buffer B: chunk 8 i + wave (cos/sin rows for chunks < 4).
template <int B, int NBUF = 3>
__device__ __forceinline__ void dma_one(const DmaConst& dc, const DmaPage& d, int i, int wave, uint32_t off) {
    const int ch = i * NWAVE + wave;
    const uint32_t m0 = ch < dc.nch ? dc.m0w + (uint32_t)(i * NWAVE * page_stride<NBUF>() + B * 1024) : dc.m0dummy;
    if (i == 0 && wave < CS_CHUNKS)
        copy16(d.rcs, m0, off);
    else
        copy16(d.rkv, m0, off);
}

template <int NLD, int B, int NBUF = 3>
__device__ __forceinline__ void dma_page(const DmaConst& dc, const PageRec& r, bool valid, int wave,
                                         const uint32_t (&doff)[NLD]) {
    const DmaPage d = dma_setup(dc, r, valid);
#pragma unroll
    for (int i = 0; i < NLD; ++i) dma_one<B, NBUF>(dc, d, i, wave, doff[i]);
}

// Copy schedule. A page's copies must reach the copy queue at about the rate the queue
// drains: a burst fills it, and a wave whose copy finds it full stalls until it has room.
// A kernel's iteration offers copy points 0 .. S::NPOS - 1 at rough positions S::time(pos)
// (fractions of the iteration). Copy c of the waves on the first wave slot of each SIMD
// (waves 0-3) goes to the point nearest c / NLD, and of the others (waves 4-7) to the
// point nearest (c + 1/2) / NLD, so that the two waves of a SIMD never issue together.
template <class S, int NLD>
constexpr int copy_point(int c, int half) {
    const float t = ((float)c + (half ? 0.5f : 0.f)) / (float)NLD;
    int best = 0;
    float bd = 2.f;
    for (int pos = 0; pos < S::NPOS; ++pos) {
        const float d = S::time(pos) > t ? S::time(pos) - t : t - S::time(pos);
        if (d < bd) {
            bd = d;
            best = pos;
        }
    }
    return best;
}

// Issues the copies of this wave that the schedule puts at copy point `pos` (a
// constant once the callers' loops are unrolled).
template <class S, int NLD, int B, int NBUF = 3>
__device__ __forceinline__ void copies_at(int pos, const DmaConst& dc, const DmaPage& d, int wave,
                                          const uint32_t (&doff)[NLD]) {
#pragma unroll
    for (int c = 0; c < NLD; ++c) {
        if (copy_point<S, NLD>(c, 0) == pos && wave < NWAVE / 2) dma_one<B, NBUF>(dc, d, c, wave, doff[c]);
        if (copy_point<S, NLD>(c, 1) == pos && wave >= NWAVE / 2) dma_one<B, NBUF>(dc, d, c, wave, doff[c]);
    }
}

// The token range of workgroup x. Workgroups are dealt to the 8 XCDs round-robin (x % 8);
// consecutive ranges, which mostly hold one request's pages, go to one XCD, so that the
// request's AB tiles are read into one L2 and shared there.
__device__ __forceinline__ int xcd_range(int x, int grid) {
    return grid % 8 == 0 ? (x % 8) * (grid / 8) + x / 8 : x;
}

// Page-loop state of a workgroup over its pages [beg, end): the page being computed j and
// the records of pages j (rc), j + 1 (r1) and j + 2 (r2; three page buffers: the page whose
// copies issue in iteration j), each loaded one iteration before it is first used. Page j
// starts a request's segment (its AB goes into registers first) when it is the range's
// first page or the request's page 0, and ends it (the partial is flushed) when it is the
// request's last page or the range's last.
struct PageLoop {
    int j, beg, end, g;
    PageRec rc, r1, r2;
};

__device__ __forceinline__ bool page_starts_seg(const PageLoop& st) { return st.j == st.beg || st.rc.k == 0; }
__device__ __forceinline__ bool page_ends_seg(const PageLoop& st) {
    return (st.rc.bits & PR_LAST) != 0 || st.j + 1 == st.end;
}

// The workgroup's page range from the header (pages per workgroup S, all pages) and the
// records of its first NBUF pages; false if the range is empty.
// S, total: the header's pages per range and page count (read by the caller beside the
// wave plan's flag, so the two loads share one latency).
template <int NBUF>
__device__ __forceinline__ bool page_loop_init(PageLoop& st, const DecodeParams& p, int g, int S, int total) {
    st.g = g;
    st.beg = min(g * S, total);
    st.end = min(st.beg + S, total);
    if (st.beg >= st.end) return false;
    st.j = st.beg;
    st.rc = page_rec(p, st.beg);
    st.r1 = st.beg + 1 < st.end ? page_rec(p, st.beg + 1) : st.rc;
    st.r2 = NBUF == 3 && st.beg + 2 < st.end ? page_rec(p, st.beg + 2) : st.r1;
    return true;
}

// End of iteration j: the records move down one page; `next` is page j + NBUF's (loaded
// during the iteration).
template <int NBUF>
__device__ __forceinline__ void page_loop_next(PageLoop& st, const PageRec& next) {
    st.rc = st.r1;
    if (NBUF == 3) {
        st.r1 = st.r2;
        st.r2 = next;
    } else {
        st.r1 = next;
    }
    ++st.j;
}

}  // namespace starkv
