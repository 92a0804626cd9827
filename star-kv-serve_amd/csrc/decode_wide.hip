// Two-pass decode for V ranks too wide for the one-pass kernels (bf16/fp16 codes with
// v_rank > 256, 3.2-bit codes with more than five 64-lane P @ V blocks), and the merge
// of its partials. decode.hip runs, per call: prep, the logits pass (the one-pass
// kernels with NB = 0: K side and softmax statistics only, every valid logit stored in
// the workspace), then `pv_kernel`, `merge_cols_kernel` and `lift_kernel` here.
//
// The reference splits its V pass the same way: logits first, then P @ V over
// column blocks of at most 512 (paged_decode.py:105-147, 199-219) or 128 channels
// inside one outlier/inlier block (paged_quant.py:311-354, 390-407).
//
// pv_kernel. Persistent workgroups whose token range g is R consecutive ranges of the
// logits pass (R = 1 unless few requests; MULTI: R > 1), partial slot (request b, range
// g) = b + g. Its reference max for request b is the largest of the logits pass's maxima
// in slots b + R g + j that hold tokens of b (merge_cols forms the same max). Per page of
// 16 tokens the workgroup copies into LDS, with buffer loads that write LDS directly (16
// bytes per lane):
//   - the V bytes of the 16 rows: bf16/fp16, the columns of the workgroup's window
//     (grid.y: windows run side by side); 3.2-bit, every V byte (scales, outlier and
//     inlier nibbles) with one window, or with several the 32 bytes holding the V scales
//     and then the window's own 32-byte chunks;
//   - the 16 logits of every head (2 KB) and the R slots' maxima per head.
// Since the reference max is final, P = exp2(logit - m) needs no rescaling.
// P @ V runs on v_mfma_f32_32x32x16 (M = 32 heads, N = 32 columns, K = the page's 16
// tokens) with A = P:
//   - bf16 codes: P = hi + lo (two bf16 parts, two MFMAs); B = 16 tokens x 32 columns
//     read with ds_read_b64_tr_b16 (a 16-lane group hands in 4 tokens x 16 columns and
//     lane i gets column i of the 4 tokens); fp16 codes: P in fp16, the same B.
//   - 3.2-bit codes: P in fp16. ds_read_b64_tr_b8 gives lane i byte-column i of 8
//     tokens, i.e. the nibbles of two V columns; the lane turns the low nibbles into
//     one fp16 B operand and the high nibbles into another (n - 8, exact), each scaled
//     by the token's V scale of its column's kind (outlier or inlier: every byte holds
//     one kind). So one 32-byte chunk of the row feeds two MFMAs, one for the even and
//     one for the odd columns of its 64. The reference folds the scale into P instead
//     (paged_quant.py:343-346); either way one product is rounded to 16 bits.
// Wave w owns the blocks (chunks) w, w + 8, ...; at the end of a request's tokens in the
// range it stores its columns of the slot's partial accumulator [Hq][ld] (fp32).
//
// LDS. Every 16-byte granule column G (8 code columns, or 16 bytes of a 3.2-bit row)
// holds the 16 tokens of a page, token t in slot t ^ (4 (G & 1)), 256 bytes per granule
// column, so 32 bf16 columns (two granule columns each way) are one 1 KB chunk and a
// transposed read of 4 tokens x 16 columns by 16 lanes touches 128 distinct bytes per
// bank group.
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
    int c_s1;        // row stride, bytes
    int n, Hq, v_rank;
    int v_off;       // byte of a row where the copied V bytes start (16-aligned)
    int ng;          // 16-byte granules copied per row
    int vs_rel;      // 3.2-bit: V scales at this byte of the copied bytes
    int vq_rel;      // 3.2-bit: first V nibble byte (outlier nibbles), relative
    int v_nout, v_nbo;  // 3.2-bit: outlier columns, their nibble bytes
    int per, units;  // window y (blockIdx.y) = units [y per, min((y + 1) per, units)): bf16/fp16,
                     // 32-column blocks (the copies start 64 y per bytes further); 3.2-bit,
                     // 32-byte chunks of the row's V bytes from v_off
    int q_u1;        // 3.2-bit: 0, one window copying every V byte (chunk c at LDS unit c); 1,
                     // several windows: unit 0 (the V scales) at LDS unit 0, the window's chunk
                     // u0 + k at LDS unit 1 + k (ng = 2 + 2 per granules copied)
    int ng_all;      // 3.2-bit: granules of V bytes in a row from v_off
    int nch;         // 1 KB chunks copied per page: logits (2), the slot's maxima (1), then V
    int nld;         // copies per wave per page
    int nbuf;        // page buffers (2 .. 8): nbuf - 1 pages in flight
    int buf_bytes;   // LDS bytes per page buffer (nch KB)
    int lds_bytes;
    uint8_t* ws; size_t ws_plan, ws_m, ws_acc, ws_lg; int lcap, acc_ld;
    int r;           // this pass's range = R consecutive logits-pass ranges
    size_t ws_pages; // page records
};


// Copy descriptors of one page (record r; valid false past the range: nothing is read):
// its rows, its logits (request b, tokens 16 k .., every head), the reference maxima of the
// R logits-pass slots b + R g + j.
struct PvPage {
    int4v_t rv, rl, rm;
};

__device__ __forceinline__ PvPage pv_page_desc(const PvParams& p, const PageRec& r, bool v, int g) {
    PvPage d;
    const int b = v ? pr_b(r.bits) : 0, k = v ? r.k : 0;
    d.rv = buffer_rsrc((const void*)(uintptr_t)r.addr, v ? pr_rows(r.bits) * p.c_s1 : 0);
    const uint8_t* lg = p.ws + p.ws_lg + (((int64_t)b * (p.lcap / TILE_TOK) + k) * p.Hq * TILE_TOK) * 4;
    d.rl = buffer_rsrc(lg, v ? p.Hq * TILE_TOK * 4 : 0);
    const uint8_t* m = p.ws + p.ws_m + (int64_t)(b + p.r * g) * p.Hq * 4;
    d.rm = buffer_rsrc(m, v ? ((p.r * p.Hq * 4 + 15) & ~15) : 0);
    return d;
}

__device__ __forceinline__ PageRec pv_rec(const PvParams& p, int j) {
    return rec_of(((crec_p)(p.ws + p.ws_pages))[j]);
}

// LDS chunks of a page buffer: 0 and 1 the logits of heads 0-15 and 16-31, 2 the R
// logits-pass slots' maxima (slot j head h at byte 4 (j Hq + h)), then the V granule
// columns.
constexpr int PV_V0 = 3;

// The copies of this wave for one page into the buffer at LDS byte `buf`: copy i moves
// chunk 8 i + wave; chunks past nch go to the dummy block and read nothing.
template <int NLD>
__device__ __forceinline__ void pv_copies(const PvParams& p, const PvPage& d, uint32_t buf, uint32_t dummy, int wave,
                                          const uint32_t (&off)[NLD]) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        if (i >= p.nld) break;
        const int ch = i * NWAVE + wave;
        const uint32_t m0 = ch < p.nch ? buf + (uint32_t)ch * 1024u : dummy;
        if (i == 0 && wave < PV_V0)
            lds_copy16(wave < 2 ? d.rl : d.rm, m0, off[i]);
        else
            lds_copy16(d.rv, m0, off[i]);
    }
}

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_t* lds_v2p;

// Byte-column (lane & 15) of 8 tokens x 16 bytes: byte e of the result is token e.
__device__ __forceinline__ uint2 tr_read8(uint32_t addr) {
    const v2i_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2p)(uintptr_t)addr);
    return make_uint2((uint32_t)r[0], (uint32_t)r[1]);
}

// fp16 (n - 8) of two nibbles: bytes x and y of w (each 0 .. 15) with fp16 1024 (0x64)
// as their high bytes, minus 1032 (all exact).
__device__ __forceinline__ half2_t nib2(uint32_t w, uint32_t sel) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, w, sel)) - (half2_t){(_Float16)1032.f, (_Float16)1032.f};
}

template <int FMT, int MB, int NLD, bool MULTI>
__global__ __launch_bounds__(NTHR) void pv_kernel(const PvParams p0) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_pv[];
    // The parameters by value: the page loop's fields stay in registers (this kernel has
    // the registers to spare) instead of being reloaded where they are used.
    const PvParams& p = p0;
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    cint_p P = (cint_p)(p.ws + 4);  // P[b]: first page of request b
    // The plan's flag and the header together (one latency), then the buffers zeroed
    // (rows past a request's end are never copied and must be finite).
    const int planned = ((cint_p)(p.ws + p.ws_plan))[NWAVE * PLAN_STRIDE];
    const int S = ((cint_p)p.ws)[0];  // pages per logits-pass range
    const int total = P[p.n];
    for (int i = tid; i < p.lds_bytes / 16; i += NTHR) ((uint4*)s_pv)[i] = make_uint4(0, 0, 0, 0);
    if (planned == 0) return;  // no plan: the merge reports NaN
    const int g = xcd_range(blockIdx.x, gridDim.x);
    const int beg = min(g * p.r * S, total), end = min(beg + p.r * S, total);
    if (beg >= end) return;
    // This workgroup's column window.
    const int u0 = (int)blockIdx.y * p.per;
    const int ncb = min(p.per, p.units - u0);
    const int c0 = FMT == FMT_Q4 ? u0 : 32 * u0;
    const int v_off = p.v_off + (FMT == FMT_Q4 ? 0 : 64 * u0);

    const uint32_t base = lds_addr(s_pv);
    const uint32_t dummy = base + (uint32_t)(p.lds_bytes - 1024);

    // Copy offsets of this lane inside a page, per copy i (chunk 8 i + wave).
    uint32_t off[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        uint32_t o = 0x80000000u;  // past every descriptor: no access
        if (ch < 2) {
            const int h = 16 * ch + (lane >> 2);
            if (h < p.Hq) o = (uint32_t)(h * 64 + 16 * (lane & 3));
        } else if (ch == 2) {
            if (4 * lane < p.r * p.Hq) o = (uint32_t)(16 * lane);
        } else if (ch < p.nch) {
            // G: the granule column in LDS; ga: the row's granule it holds (same parity).
            const int G = 4 * (ch - PV_V0) + (lane >> 4), t = gslot(G, lane & 15);
            const int ga = FMT == FMT_Q4 && p.q_u1 && G >= 2 ? G - 2 + 2 * u0 : G;
            if (G < p.ng && (FMT != FMT_Q4 || ga < p.ng_all)) o = (uint32_t)(t * p.c_s1 + v_off + 16 * ga);
        }
        off[i] = o;
    }

    // A operand: head am = lane & 31, tokens 8 ag .. 8 ag + 7 (ag = lane >> 5).
    const int am = lane & 31, ag = lane >> 5;
    // B operand reads of block (or chunk) 0, relative to the page buffer.
    uint32_t trd0, trd1;
    {
        const int q = lane >> 4, i = lane & 15;
        if (FMT == FMT_Q4) {
            // 16-lane group q: granule 2 c + (q & 1), tokens 8 (q >> 1) + i / 2, bytes 8 (i & 1).
            const int G = q & 1, t = 8 * (q >> 1) + (i >> 1);
            trd0 = (uint32_t)((G * 16 + gslot(G, t)) * 16 + 8 * (i & 1));
            trd1 = 0;
        } else {
            // tokens 8 (q >> 1) + i / 4 (+ 4), columns 16 (q & 1) + 4 (i % 4).
            const int t = 8 * (q >> 1) + (i >> 2);
            const int col = 16 * (q & 1) + 4 * (i & 3);
            const int G = col >> 3, h = (col >> 2) & 1;
            trd0 = (uint32_t)((G * 16 + gslot(G, t)) * 16 + 8 * h);
            trd1 = (uint32_t)((G * 16 + gslot(G, t + 4)) * 16 + 8 * h);
        }
    }
    const uint32_t lga = (uint32_t)((am * 16 + 8 * ag) * 4);  // logits of (am, 8 ag ..)
    const uint32_t mxa = (uint32_t)(2 * 1024 + am * 4);         // slot 0's max of head am
    __syncthreads();

    f32x16_t acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (f32x16_t){};

    // Records: the current page j (cur), j + 1 (ncur, loaded in iteration j), the page whose
    // copies issue in iteration j (cpy = page j + nbuf - 1, loaded in iteration j - 1).
    PageRec cur = pv_rec(p, beg);
    // Prologue: pages beg .. beg + nbuf - 2 in flight.
    for (int j = 0; j < p.nbuf - 1; ++j) {
        const bool v = beg + j < end;
        const PageRec r = v ? pv_rec(p, beg + j) : cur;
        pv_copies<NLD>(p, pv_page_desc(p, r, v, g), base + (uint32_t)(j * p.buf_bytes), dummy, wave, off);
    }
    int jc = beg + p.nbuf - 1;  // the page whose copies issue next
    PageRec cpy = jc < end ? pv_rec(p, jc) : cur;
    int jb = 0;  // buffer of the current page
    // The logits-pass ranges R g + j holding pages of request b: bit j. This pass's
    // reference max of the request is the largest of theirs (slots of other ranges hold
    // other requests' values, or none).
    auto sub_mask = [&](int b) -> int {
        if (!MULTI) return 1;  // R = 1: the one range is this workgroup's
        const int lo = P[b], hi = P[b + 1];
        int msk = 0;
        for (int j = 0; j < p.r; ++j) {
            const int r0 = (p.r * g + j) * S;
            if (max(r0, lo) < min(r0 + S, hi)) msk |= 1 << j;
        }
        return msk;
    };
    int msk = sub_mask(pr_b(cur.bits));  // of the current request, redone when the request changes
    for (int j = beg; j < end; ++j) {
        // Page j is in buffer jb; the copies of the nbuf - 2 pages after it may still run.
        wait_vmcnt_lgkm0_wide((p.nbuf - 2) * p.nld);
        wait_lgkm0_barrier();  // every wave is done with the previous page's buffer
        {
            const int jn = jb == 0 ? p.nbuf - 1 : jb - 1;  // the buffer the previous page used
            pv_copies<NLD>(p, pv_page_desc(p, cpy, jc < end, g), base + (uint32_t)(jn * p.buf_bytes), dummy, wave,
                           off);
        }
        // The records of the next iteration: they arrive under its wait.
        ++jc;
        const PageRec ncpy = jc < end ? pv_rec(p, jc) : cur;
        const PageRec ncur = j + 1 < end ? pv_rec(p, j + 1) : cur;
        const int rows = pr_rows(cur.bits);
        const uint32_t buf = base + (uint32_t)(jb * p.buf_bytes);
        const uint32_t vbuf = buf + PV_V0 * 1024;  // the page's V granule columns
        // A operand: P of head am at tokens 8 ag .. 8 ag + 7 of this page.
        const f32x4_t s0 = lds_ld<f32x4_t>(buf + lga), s1 = lds_ld<f32x4_t>(buf + lga + 16);
        // R = 1: the slot's max. Else the largest of the R slots' maxima (all four read:
        // the slots past R are in the chunk too), those of other requests' ranges left out.
        float mx;
        if constexpr (MULTI) {
            mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float mj = lds_ld<float>(buf + mxa + (uint32_t)(4 * j * p.Hq));
                mx = (msk >> j) & 1 ? fmaxf(mx, mj) : mx;
            }
        } else {
            mx = lds_ld<float>(buf + mxa);
        }
        const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const int tok0 = 8 * ag;  // this lane's first token in the page
        float pe[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool ok = am < p.Hq && tok0 + e < rows;
            pe[e] = __builtin_amdgcn_exp2f(ok ? sv[e] - mx : -INFINITY);  // no branch: exp2(-inf) = 0
        }
        if constexpr (FMT == FMT_BF16) {
            float lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) lo[e] = pe[e] - (float)(__bf16)pe[e];
            const bf16x8_t ahi = to_bf16x8(pe), alo = to_bf16x8(lo);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int cb = wave + NWAVE * i;
                if (cb < ncb) {
                    const uint32_t a = vbuf + (uint32_t)cb * 1024u;
                    const uint2 b0 = tr_read(a + trd0), b1 = tr_read(a + trd1);
                    const bf16x8_t bv = __builtin_bit_cast(bf16x8_t, make_uint4(b0.x, b0.y, b1.x, b1.y));
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi, bv, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo, bv, acc[i], 0, 0, 0);
                }
            }
        } else if constexpr (FMT == FMT_F16) {
            const half8_t av = to_f16x8(pe);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int cb = wave + NWAVE * i;
                if (cb < ncb) {
                    const uint32_t a = vbuf + (uint32_t)cb * 1024u;
                    const uint2 b0 = tr_read(a + trd0), b1 = tr_read(a + trd1);
                    const half8_t bv = __builtin_bit_cast(half8_t, make_uint4(b0.x, b0.y, b1.x, b1.y));
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i], 0, 0, 0);
                }
            }
        } else {
            const half8_t av = to_f16x8(pe);
            // This lane's 8 tokens' V scales as fp16 pairs (tokens 2j, 2j + 1), per kind.
            uint32_t so[4], si[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 8 * ag + 2 * j;
                const uint32_t w0 = lds_ld<uint32_t>(vbuf + (uint32_t)(gslot(0, t) * 16 + p.vs_rel));
                const uint32_t w1 = lds_ld<uint32_t>(vbuf + (uint32_t)(gslot(0, t + 1) * 16 + p.vs_rel));
                so[j] = h2_bits(cvt_h2(__uint_as_float(w0 << 16), __uint_as_float(w1 << 16)));
                si[j] = h2_bits(cvt_h2(__uint_as_float(w0 & 0xffff0000u), __uint_as_float(w1 & 0xffff0000u)));
            }
            // Every chunk's bytes first (chunks past the window reread the last one, unused).
            uint2 wv[MB / 2];
#pragma unroll
            for (int i = 0; i < MB / 2; ++i)
                wv[i] = tr_read8(vbuf + (uint32_t)((p.q_u1 ? 1 : c0) + min(wave + NWAVE * i, ncb - 1)) * 512u + trd0);
#pragma unroll
            for (int i = 0; i < MB / 2; ++i) {
                const int ch = wave + NWAVE * i;  // 32-byte chunk of the copied V bytes
                if (ch < ncb) {
                    const int c = c0 + ch;
                    const uint2 w = wv[i];
                    // This lane's byte: outlier columns before v_nbo bytes of nibbles, inlier after.
                    const bool inl = 32 * c + (lane & 31) - p.vq_rel >= p.v_nbo;
                    const uint32_t l0 = w.x & 0x0F0F0F0Fu, l1 = w.y & 0x0F0F0F0Fu;
                    const uint32_t h0 = (w.x >> 4) & 0x0F0F0F0Fu, h1 = (w.y >> 4) & 0x0F0F0F0Fu;
                    half2_t sc[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) sc[j] = as_h2(inl ? si[j] : so[j]);
                    const half2_t e0 = nib2(l0, 0x04010400u) * sc[0], e1 = nib2(l0, 0x04030402u) * sc[1];
                    const half2_t e2 = nib2(l1, 0x04010400u) * sc[2], e3 = nib2(l1, 0x04030402u) * sc[3];
                    const half2_t o0 = nib2(h0, 0x04010400u) * sc[0], o1 = nib2(h0, 0x04030402u) * sc[1];
                    const half2_t o2 = nib2(h1, 0x04010400u) * sc[2], o3 = nib2(h1, 0x04030402u) * sc[3];
                    const half8_t be = __builtin_bit_cast(
                        half8_t, make_uint4(h2_bits(e0), h2_bits(e1), h2_bits(e2), h2_bits(e3)));
                    const half8_t bo = __builtin_bit_cast(
                        half8_t, make_uint4(h2_bits(o0), h2_bits(o1), h2_bits(o2), h2_bits(o3)));
                    acc[2 * i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, be, acc[2 * i], 0, 0, 0);
                    acc[2 * i + 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bo, acc[2 * i + 1], 0, 0, 0);
                }
            }
        }
        const bool seg_end = (cur.bits & PR_LAST) != 0 || j + 1 == end;
        if (seg_end) {
            // This lane's column of each of its blocks, for the 16 heads
            // 8 (j / 4) + 4 (lane >> 5) + j % 4 of the 32x32 result.
            const int64_t slot = (int64_t)pr_b(cur.bits) + g;
            float* wa = (float*)(p.ws + p.ws_acc) + slot * p.Hq * p.acc_ld;
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                int col = -1;
                if (FMT == FMT_Q4) {
                    const int ch = wave + NWAVE * (i >> 1);
                    const int rel = 32 * (c0 + ch) + (lane & 31) - p.vq_rel;  // nibble byte of this lane
                    if (ch < ncb && rel >= 0) {
                        if (rel < p.v_nbo) {
                            col = 2 * rel + (i & 1);
                            if (col >= p.v_nout) col = -1;
                        } else {
                            col = p.v_nout + 2 * (rel - p.v_nbo) + (i & 1);
                        }
                    }
                } else {
                    const int cb = wave + NWAVE * i;
                    if (cb < ncb) col = c0 + 32 * cb + (lane & 31);
                }
                const bool okc = col >= 0 && col < p.v_rank;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int h = 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
                    if (okc && h < p.Hq) wa[(int64_t)h * p.acc_ld + col] = acc[i][j];
                    acc[i][j] = 0.f;
                }
            }
        }
        cur = ncur;
        cpy = ncpy;
        if (MULTI && seg_end && j + 1 < end) msk = sub_mask(pr_b(cur.bits));
        jb = jb + 1 == p.nbuf ? 0 : jb + 1;
    }
    wait_vmcnt_lgkm0(0);  // no copy may land after the workgroup ends
}

// ---------------------------------------------------------------------------
// Merge of the two-pass partials, in two launches.
// merge_cols_kernel<MCW, U>: one workgroup per (request, head, column block): the
//   log-sum-exp weights of the request's slots (the first 256 kept in registers), then each
//   column's weighted sum of their accumulators, U partials' loads in flight, divided by the
//   total, into o [n][Hq][ld] (NaN for a request with no tokens, as the reference's softmax
//   over an empty row). MCW = 1: the four waves take different columns (1024 per
//   workgroup), each over every slot; MCW = 8 (eight waves), for requests split over many
//   workgroups (a few long requests): wave w sums slots w, w + 8, ... of 256 columns, then
//   the waves' sums are added.
// lift_kernel<DT, REQ, THR, DQ>: one workgroup per (head, REQ requests, 8 DQ output
//   columns): out = o @ v_up_by_q[h], each thread 8 output columns over a THR / DQ-th of the
//   rank columns, LIFT_U rows in flight, then a reduction over those parts. 8 requests x
//   512 threads x all 128 columns; for at most 8 requests, 2 x 1024 threads x 32 columns
//   (four workgroups per head and request pair: one request's v_up_by_q rows are read by
//   128 workgroups instead of 32).
// ---------------------------------------------------------------------------
constexpr int MC_THR = 256;
constexpr int MC_WREG = 4;  // slot weights held in registers: 64 MC_WREG slots
constexpr int LIFT_U = 8;   // v_up_by_q rows per thread in flight

template <int MCW, int U, int THR>
__global__ __launch_bounds__(THR) void merge_cols_kernel(const uint8_t* __restrict__ ws, size_t ws_plan, size_t ws_m,
                                                            size_t ws_l, size_t ws_acc, size_t ws_o, int n, int Hq,
                                                            int v_rank, int ld, int pv_r) {
    constexpr int CPW = 4 * THR / MCW;  // columns per workgroup
    __shared__ f32x4_t s_sum[MCW][64];
    __shared__ float s_mr[64 * MC_WREG];  // R > 1: the slots' maxima held in registers, for reads by index
    const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int w = MCW > 1 ? __builtin_amdgcn_readfirstlane(tid >> 6) : 0;  // slot phase
    const int* hdr = (const int*)ws;
    const float* wm = (const float*)(ws + ws_m);
    const float* wl = (const float*)(ws + ws_l);
    const float* wa = (const float*)(ws + ws_acc);
    const int SL = hdr[0];        // tokens per logits-pass range
    const int S = SL * pv_r;      // tokens per P @ V range
    const bool planned = ((const int*)(ws + ws_plan))[NWAVE * PLAN_STRIDE] != 0;
    const int pb = hdr[1 + b], pe = hdr[2 + b];
    const bool live = pe > pb && S > 0 && planned;
    // The request's logits-pass slots b + r_lo + i (i < nr) and P @ V slots b + k_lo + k (k < nk).
    const int r_lo = live ? pb / SL : 0, nr = live ? (pe - 1) / SL - r_lo + 1 : 0;
    const int k_lo = live ? pb / S : 0, nk = live ? (pe - 1) / S - k_lo + 1 : 0;
    const int64_t s0 = (int64_t)(k_lo + b) * Hq + h;  // P @ V slot row of partial k: s0 + k Hq
    const int64_t r0 = (int64_t)(r_lo + b) * Hq + h;  // logits-pass slot row i: r0 + i Hq
    // Every wave forms the same weights (the loads hit the same lines): the request's max M
    // and sum l over its logits-pass slots; P @ V partial k weighs 2^(M_k - M), M_k its
    // reference max: the largest of the logits-pass maxima of its range's R slots that
    // hold tokens of the request (as the P @ V pass formed it). The first 64 MC_WREG
    // logits-pass slots' maxima are held in registers (slot i in lane i % 64 of mr[i / 64]),
    // and so are the weights of the first 64 MC_WREG partials (wk).
    float mr[MC_WREG], lr[MC_WREG];
#pragma unroll
    for (int j = 0; j < MC_WREG; ++j) {
        const int i = lane + 64 * j;
        mr[j] = i < nr ? wm[r0 + (int64_t)i * Hq] : -INFINITY;
        lr[j] = i < nr ? wl[r0 + (int64_t)i * Hq] : 0.f;
    }
    float M = mr[0];
#pragma unroll
    for (int j = 1; j < MC_WREG; ++j) M = fmaxf(M, mr[j]);
    for (int i = lane + 64 * MC_WREG; i < nr; i += 64) M = fmaxf(M, wm[r0 + (int64_t)i * Hq]);
    M = wave_max(M);
    float l = 0.f;
#pragma unroll
    for (int j = 0; j < MC_WREG; ++j) l = fmaf(lr[j], lane + 64 * j < nr ? exp2f(mr[j] - M) : 0.f, l);
    for (int i = lane + 64 * MC_WREG; i < nr; i += 64) {
        const int64_t sl = r0 + (int64_t)i * Hq;
        l += wl[sl] * exp2f(wm[sl] - M);
    }
    l = wave_sum(l);
    // M_k from memory (partials past 64 MC_WREG, under divergent lanes).
    auto slot_max = [&](int k) -> float {
        float x = -INFINITY;
        for (int t = 0; t < pv_r; ++t) {
            const int i = pv_r * (k_lo + k) + t - r_lo;
            if (i >= 0 && i < nr) x = fmaxf(x, wm[r0 + (int64_t)i * Hq]);
        }
        return x;
    };
    float wk[MC_WREG];
    if (pv_r == 1) {  // partial k is logits-pass slot k
#pragma unroll
        for (int j = 0; j < MC_WREG; ++j) wk[j] = lane + 64 * j < nk ? exp2f(mr[j] - M) : 0.f;
    } else {  // the maxima by slot index from LDS (every wave formed the same; wave 0 stores them)
        if (tid < 64) {
#pragma unroll
            for (int j = 0; j < MC_WREG; ++j) s_mr[lane + 64 * j] = mr[j];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MC_WREG; ++j) {
            const int k = lane + 64 * j;
            float x = -INFINITY;
            for (int t = 0; t < pv_r; ++t) {
                const int i = pv_r * (k_lo + k) + t - r_lo;
                const float v = i < 0 || i >= nr           ? -INFINITY
                                : i < 64 * MC_WREG ? s_mr[i]
                                                   : wm[r0 + (int64_t)i * Hq];
                x = fmaxf(x, v);
            }
            wk[j] = k < nk ? exp2f(x - M) : 0.f;
        }
    }
    const float inv = live ? 1.f / l : __builtin_nanf("");
    float* o = (float*)(ws + ws_o) + ((int64_t)b * Hq + h) * ld;
    const int c4 = blockIdx.z * CPW + 4 * (MCW > 1 ? lane : tid);
    // Weight of slot k (wave-uniform k). The lane reads come from wk as formed above, with
    // every lane active (inside the column branch below some lanes are not).
    auto weight = [&](int k) -> float {
        if (k < 64 * MC_WREG) {
            float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wk[0]), k & 63));
#pragma unroll
            for (int j = 1; j < MC_WREG; ++j)
                if (k >= 64 * j) x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wk[j]), k & 63));
            return x;
        }
        return exp2f(slot_max(k) - M);
    };
    f32x4_t a = {0.f, 0.f, 0.f, 0.f};
    if (c4 < v_rank) {
        int k = w;  // wave-uniform
        for (; k + (U - 1) * MCW < nk; k += U * MCW) {  // U partials' loads in flight
            f32x4_t r[U];
#pragma unroll
            for (int u = 0; u < U; ++u) r[u] = *(const f32x4_t*)(wa + (s0 + (int64_t)(k + u * MCW) * Hq) * ld + c4);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int ku = k + u * MCW;
                a += r[u] * weight(ku);
            }
        }
        for (; k < nk; k += MCW) {
            const int64_t sl = s0 + (int64_t)k * Hq;
            a += *(const f32x4_t*)(wa + sl * ld + c4) * weight(k);
        }
    }
    if constexpr (MCW == 1) {
        if (c4 < v_rank) *(f32x4_t*)(o + c4) = a * inv;
    } else {
        s_sum[w][lane] = a;
        __syncthreads();
        if (w == 0 && c4 < v_rank) {
            f32x4_t t = s_sum[0][lane];
#pragma unroll
            for (int k = 1; k < MCW; ++k) t += s_sum[k][lane];
            *(f32x4_t*)(o + c4) = t * inv;
        }
    }
}

template <int DT, int LIFT_REQ, int LIFT_THR, int DQ>
__global__ __launch_bounds__(LIFT_THR) void lift_kernel(const uint8_t* __restrict__ ws, size_t ws_o, int n, int Hq,
                                                        int v_rank, int ld, const void* __restrict__ vup,
                                                        int64_t vu_s0, int64_t vu_s1, void* __restrict__ out,
                                                        int64_t o_s0, int64_t o_s1, int out_dt) {
    static_assert(DQ == 16 || DQ == 4, "8 DQ output columns per workgroup: 128 or 32");
    constexpr int LIFT_WAVES = LIFT_THR / 64;
    constexpr int DW = 8 * DQ;  // output columns of this workgroup
    extern __shared__ __align__(16) uint8_t s_dyn[];
    float* s_o = (float*)s_dyn;    // [LIFT_REQ][ld]
    float* s_red = (float*)s_dyn;  // [LIFT_WAVES][LIFT_REQ][DW], over s_o once the products are done
    const int h = blockIdx.x, b0 = blockIdx.y * LIFT_REQ;  // head in x: a head's workgroups share one XCD's L2
    const int d0 = blockIdx.z * DW;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* og = (const float*)(ws + ws_o);
    // Thread (dq, cp): output columns d0 + 8 dq .. + 7 over rank columns c = cp (mod CP);
    // LIFT_U rows of v_up_by_q are loaded before their products, so their latencies overlap
    // (the first LIFT_U before the rows o are staged).
    constexpr int CP = LIFT_THR / DQ;
    const int dq = tid % DQ, cp = tid / DQ;
    const int64_t vh = (int64_t)h * vu_s0 + d0 + 8 * dq;
    float u[LIFT_U][8];
    auto load_rows = [&](int c0) {
#pragma unroll
        for (int j = 0; j < LIFT_U; ++j) {
            const int c = min(c0 + CP * j, v_rank - 1);  // past the end: a valid row, weighted 0 below
            load8_f(vup, vh + (int64_t)c * vu_s1, DT, u[j]);
        }
    };
    load_rows(cp);
    for (int i = 4 * tid; i < LIFT_REQ * ld; i += 4 * LIFT_THR) {
        const int r = i / ld, c = i - r * ld;
        f32x4_t v = {0.f, 0.f, 0.f, 0.f};
        if (b0 + r < n) v = *(const f32x4_t*)(og + ((int64_t)(b0 + r) * Hq + h) * ld + c);
        *(f32x4_t*)(s_o + i) = v;
    }
    __syncthreads();
    float acc[LIFT_REQ][8];
#pragma unroll
    for (int r = 0; r < LIFT_REQ; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
    for (int c0 = cp; c0 < v_rank; c0 += CP * LIFT_U) {
        if (c0 != cp) load_rows(c0);
#pragma unroll
        for (int j = 0; j < LIFT_U; ++j) {
            const int c = c0 + CP * j;
#pragma unroll
            for (int r = 0; r < LIFT_REQ; ++r) {
                const float x = c < v_rank ? s_o[r * ld + c] : 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r][e] = fmaf(x, u[j][e], acc[r][e]);
            }
        }
    }
    // Sum over the lanes of the wave with the same dq (lane = dq + DQ k): for DQ = 4 first
    // over lanes l, l ^ 4, l ^ 8, l ^ 12 of each row (row rotations by 8 and 4), then over
    // the four rows; then over the waves.
#pragma unroll
    for (int r = 0; r < LIFT_REQ; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[r][e];
            if constexpr (DQ == 4) {
                v += dpp_f<0x128>(v);  // row_ror:8
                v += dpp_f<0x124>(v);  // row_ror:4
            }
            acc[r][e] = sum_rows(v);
        }
    __syncthreads();  // every wave is done with s_o
    if (lane < DQ) {
#pragma unroll
        for (int r = 0; r < LIFT_REQ; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e) s_red[(w * LIFT_REQ + r) * DW + 8 * dq + e] = acc[r][e];
    }
    __syncthreads();
    for (int i = tid; i < LIFT_REQ * DW; i += LIFT_THR) {
        const int r = i / DW, d = i % DW, b = b0 + r;
        if (b >= n) continue;
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < LIFT_WAVES; ++k) v += s_red[(k * LIFT_REQ + r) * DW + d];
        store_f(out, (int64_t)b * o_s0 + (int64_t)h * o_s1 + d0 + d, out_dt, v);
    }
}

// ---------------------------------------------------------------------------
// Host side of the P @ V pass and the merge.
// ---------------------------------------------------------------------------
namespace {

constexpr int PV_NLD = 12;  // copies per wave per page, at most (the plan keeps nch <= 96)
// Page bytes in flight per workgroup the plan aims for, with at least two pages in flight.
// A page costs about the same time whatever its width (its barrier, P and copy issue), so
// the plan takes the fewest windows that keep this much in flight: at V rank 1280 one
// window of 40 blocks (86 KB in flight) runs 64 x 8192 in 286 us where two windows of 20
// (115 KB) took 346 us.
constexpr int PV_INFLIGHT = 64 * 1024;

template <int FMT, bool MULTI>
const void* pv_pick(int mb) {
    if (mb <= 2) return (const void*)&pv_kernel<FMT, 2, PV_NLD, MULTI>;
    if (mb <= 4) return (const void*)&pv_kernel<FMT, 4, PV_NLD, MULTI>;
    if (mb <= 6) return (const void*)&pv_kernel<FMT, 6, PV_NLD, MULTI>;
    return (const void*)&pv_kernel<FMT, 8, PV_NLD, MULTI>;
}

template <int FMT>
const void* pv_pick_r(int mb, int r) {
    return r > 1 ? pv_pick<FMT, true>(mb) : pv_pick<FMT, false>(mb);
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

// Dynamic LDS of lift_kernel<DT, req, thr, dq>: the rows o [req][ld], then (over them)
// the per-wave sums [thr / 64][req][8 dq].
size_t lift_lds(int ld, int req = 8, int thr = 512, int dq = 16) {
    return std::max((size_t)req * ld * 4, (size_t)(thr / 64) * req * 8 * dq * 4);
}

}  // namespace

// The plan of the P @ V pass: units (32-column blocks of bf16/fp16 codes, 32-byte chunks
// of the copied 3.2-bit V bytes) per launch, at most 8 per wave's accumulators (64
// MFMA blocks), and the LDS geometry.
struct PvPlan {
    int units;      // in all
    int per;        // per window
    int nbuf, nch, nld, lds;
    int ng, v_off;  // copy geometry: granules copied per row (of one window) and the first byte
    int ng_all;     // 3.2-bit: granules of V bytes per row
    int q_u1;       // 3.2-bit: several windows (each copies unit 0, the V scales, then its own units)
    bool ok;
};

// min_windows: at least this many column windows, when each can keep 4 units.
// v_col (bf16/fp16): the first V lane of a row.
static PvPlan pv_plan(int fmt, int v_col, int v_rank, int vs_off, int vq_off, int v_bytes, int min_windows = 1) {
    PvPlan pl{};
    int max_units;
    if (fmt == FMT_Q4) {
        pl.v_off = vs_off & ~15;
        pl.ng_all = (vq_off + v_bytes + 15) / 16 - pl.v_off / 16;
        pl.units = (pl.ng_all + 1) / 2;
        max_units = 32;  // 2 blocks each
    } else {
        pl.v_off = 2 * v_col;
        pl.units = (v_rank + 31) / 32;
        max_units = 64;
    }
    // Fewest windows (each re-reads the logits) whose pages keep at least PV_INFLIGHT
    // bytes in flight per workgroup, else the most bytes in flight.
    int lo = (pl.units + std::min(pl.units, max_units) - 1) / std::min(pl.units, max_units);
    lo = std::max(lo, std::min(min_windows, pl.units / 4));
    int best_score = -1;
    for (int launches = lo; launches <= lo + 3; ++launches) {
        const int per = (pl.units + launches - 1) / launches;
        if (per > max_units) continue;
        // 3.2-bit windows copy unit 0 (the V scales) and their own units.
        const bool q_win = fmt == FMT_Q4 && per < pl.units;
        const int ng = fmt == FMT_Q4 ? (q_win ? 2 + 2 * per : pl.ng_all) : 4 * per;
        const int nch = (ng + 3) / 4 + PV_V0;
        if ((nch + NWAVE - 1) / NWAVE > PV_NLD) continue;
        const int nbuf = std::min(8, (PV_MAX_DYN_LDS - 1024) / (nch * 1024));
        if (nbuf < 2) continue;
        const int inflight = (nbuf - 1) * nch * 1024;
        const int score = inflight >= PV_INFLIGHT && nbuf >= 3 ? (1 << 30) - launches : inflight;
        if (score > best_score) {
            best_score = score;
            pl.per = per;
            pl.nbuf = nbuf;
            pl.nch = nch;
            pl.nld = (nch + NWAVE - 1) / NWAVE;
            pl.lds = nbuf * nch * 1024 + 1024;
            pl.ng = ng;
            pl.q_u1 = q_win ? 1 : 0;
            pl.ok = true;
        }
    }
    return pl;
}

int launch_pv(const DecodeParams& p, int fmt, int grid, hipStream_t stream) {
    const int v_bytes = p.v_nbo + (p.v_rank - p.v_nout + 1) / 2;
    // A grid short of the CUs (few requests) takes more, narrower windows side by side.
    const int cus = device_cus();
    const int gp = (grid + p.pv_r - 1) / p.pv_r;  // this pass's ranges
    PvPlan pl = pv_plan(fmt, p.v_col, p.v_rank, p.vs_off, p.vq_off, v_bytes, (cus + gp - 1) / gp);
    if (!pl.ok) pl = pv_plan(fmt, p.v_col, p.v_rank, p.vs_off, p.vq_off, v_bytes);
    SKV_CHECK(pl.ok, "decode: no P @ V window fits in LDS (v_rank %d)", p.v_rank);
    PvParams a;
    memset(&a, 0, sizeof(a));
    a.c_s1 = (int)p.c_s1;
    a.n = p.n; a.Hq = p.Hq; a.v_rank = p.v_rank;
    a.ng = pl.ng;
    a.ng_all = pl.ng_all;
    a.q_u1 = pl.q_u1;
    a.vs_rel = p.vs_off - pl.v_off;
    a.vq_rel = p.vq_off - pl.v_off;
    a.v_nout = p.v_nout; a.v_nbo = p.v_nbo;
    a.nch = pl.nch; a.nld = pl.nld; a.nbuf = pl.nbuf; a.buf_bytes = pl.nch * 1024;
    a.lds_bytes = pl.lds;
    a.ws = p.ws; a.ws_plan = p.ws_plan; a.ws_m = p.ws_m; a.ws_acc = p.ws_acc; a.ws_lg = p.ws_lg; a.lcap = p.lcap;
    a.acc_ld = p.acc_ld;
    a.r = p.pv_r;
    a.ws_pages = p.ws_pages;
    // The windows run side by side in one launch (grid.y): each re-reads the page logits.
    a.per = pl.per;
    a.units = pl.units;
    a.v_off = pl.v_off;
    const int windows = (pl.units + pl.per - 1) / pl.per;
    const int mb = fmt == FMT_Q4 ? 2 * ((pl.per + NWAVE - 1) / NWAVE) : (pl.per + NWAVE - 1) / NWAVE;
    const void* fn = fmt == FMT_BF16 ? pv_pick_r<FMT_BF16>(mb, p.pv_r)
                     : fmt == FMT_F16 ? pv_pick_r<FMT_F16>(mb, p.pv_r)
                                      : pv_pick_r<FMT_Q4>(mb, p.pv_r);
    int rc = raise_lds(fn, PV_MAX_DYN_LDS);
    if (rc) return rc;
    void* args[] = {(void*)&a};
    SKV_HIP(hipLaunchKernel(fn, dim3(gp, windows), dim3(NTHR), args, (size_t)a.lds_bytes, stream));
    return STARKV_OK;
}

bool pv_fits(int fmt, int k_width, int v_rank, int vs_off, int vq_off, int v_nout, int v_bytes) {
    (void)v_nout;
    return pv_plan(fmt, k_width, v_rank, vs_off, vq_off, v_bytes).ok &&
           lift_lds((v_rank + 3) & ~3) <= (size_t)PV_MAX_DYN_LDS;
}

int launch_merge_wide(const DecodeParams& p, int grid, int w_dt, const void* vup, int64_t vu_s0, int64_t vu_s1,
                      void* out, int64_t o_s0, int64_t o_s1, int out_dt, hipStream_t stream) {
    const size_t lds = lift_lds(p.acc_ld);
    SKV_CHECK(lds <= (size_t)PV_MAX_DYN_LDS, "decode: v_rank %d too large for the merge", p.v_rank);
    // Slots per request: about gp / n + 1. Many (a few long requests): split them over waves.
    const int gp = (grid + p.pv_r - 1) / p.pv_r;
    if (gp >= 8 * p.n)
        hipLaunchKernelGGL((merge_cols_kernel<16, 8, 1024>), dim3(p.n, p.Hq, (p.v_rank + 255) / 256), dim3(1024), 0,
                           stream, (const uint8_t*)p.ws, p.ws_plan, p.ws_m, p.ws_l, p.ws_acc, p.ws_o, p.n, p.Hq,
                           p.v_rank, p.acc_ld, p.pv_r);
    else
        hipLaunchKernelGGL((merge_cols_kernel<1, 8, MC_THR>), dim3(p.n, p.Hq, (p.v_rank + 1023) / 1024), dim3(MC_THR), 0,
                           stream, (const uint8_t*)p.ws, p.ws_plan, p.ws_m, p.ws_l, p.ws_acc, p.ws_o, p.n, p.Hq,
                           p.v_rank, p.acc_ld, p.pv_r);
    SKV_HIP(hipGetLastError());
    const bool small = p.n <= 8;
    const int req = small ? 2 : 8, thr = small ? 1024 : 512, dq = small ? 4 : 16;
    const void* fn = small ? (w_dt == STARKV_BF16 ? (const void*)&lift_kernel<STARKV_BF16, 2, 1024, 4>
                              : w_dt == STARKV_F16 ? (const void*)&lift_kernel<STARKV_F16, 2, 1024, 4>
                                                   : (const void*)&lift_kernel<STARKV_F32, 2, 1024, 4>)
                           : (w_dt == STARKV_BF16 ? (const void*)&lift_kernel<STARKV_BF16, 8, 512, 16>
                              : w_dt == STARKV_F16 ? (const void*)&lift_kernel<STARKV_F16, 8, 512, 16>
                                                   : (const void*)&lift_kernel<STARKV_F32, 8, 512, 16>);
    int rc = raise_lds(fn, PV_MAX_DYN_LDS);
    if (rc) return rc;
    const size_t lds2 = lift_lds(p.acc_ld, req, thr, dq);
    SKV_CHECK(lds2 <= (size_t)PV_MAX_DYN_LDS, "decode: v_rank %d too large for the lift", p.v_rank);
    const uint8_t* ws = p.ws;
    size_t wo = p.ws_o;
    int n = p.n, Hq = p.Hq, vr = p.v_rank, ld = p.acc_ld;
    void* args[] = {(void*)&ws, (void*)&wo, (void*)&n, (void*)&Hq, (void*)&vr, (void*)&ld, (void*)&vup,
                    (void*)&vu_s0, (void*)&vu_s1, (void*)&out, (void*)&o_s0, (void*)&o_s1, (void*)&out_dt};
    SKV_HIP(hipLaunchKernel(fn, dim3(p.Hq, (p.n + req - 1) / req, 128 / (8 * dq)), dim3(thr), args, lds2, stream));
    return STARKV_OK;
}

}  // namespace starkv
