// 3.2-bit paged decode: the decode launch of starkv_quant_decode (decode.hip holds the
// setup, fold and merge launches and the host entry points).
//
// The page walk is the one of the bf16/fp16 kernel (decode_lowrank.hip): one persistent
// workgroup of 8 waves per CU over a contiguous token range, three page buffers
// interleaved at 1 KB, copies spread over the iteration, whole query heads per wave with
// their AB tiles (q folded into U) in VGPRs, z = AB . [cos|sin]^T on MFMA. What differs
// is the row format (paged_quant.py:71-111: K nibbles, per-head (outlier, inlier) bf16
// K scales, (outlier, inlier) bf16 V scales, V nibbles with the outlier columns first)
// and with it both sides of the page:
//
// K side. The 4 z values a lane receives for a tile are ranks (2g, 2g+8, 2g+1, 2g+9),
// g = lane >> 4 (the fold orders AB so and scales the last two by 1/16). Their codes
// are the low and high nibbles of bytes g and g+4 of the tile's 8 code bytes: one byte
// permute moves both bytes into one word, one and-or each builds the fp16 pairs
// 1024 + n (low nibbles) and 1024 + 16 n (high nibbles), and one packed subtract each
// gives (n - 8) and 16 (n - 8), all exact. The scales are per (token, head), so the
// tiles leave them out: each tile's lanes produce the unscaled dot d, and a head's first
// tile, which holds its outlier ranks (the first nout of the head, paged_quant.py:
// 298-300), also the dot over the outlier ranks alone, e. The softmax then forms
// logit = s_in * sum(d) + (s_out - s_in) * e once per (head, token).
//
// V side. The per-token V scales are folded into P, as the reference does
// (paged_quant.py:346): the softmax writes P * s_out and P * s_in, and each P @ V lane
// reads the one its column needs (the 4x4x4 MFMA's A operand is per 4-lane block here,
// not broadcast). Lane-entries L < O4 (v_nout rounded up to 4, so no block mixes the two
// kinds) hold outlier column L; the rest hold inlier column v_nout + L - O4. The V
// nibbles of a page are expanded once per workgroup, every thread two lane-entries of
// one token, into an fp16 table in the B-operand layout; the table becomes visible at
// the next page's barrier, so iteration j runs the K side and softmax of page j and
// P @ V of page j - 1.
//
// LDS chunks of a page buffer (see decode_pages.hpp for the interleave):
//   0 .. 3                cos/sin rows
//   4 .. nch - 1          the rows, 16-byte granule column G (16 rows x 16 B) at
//                         chunk 4 + G / 4, offset (G % 4) * 256, row t at +16 t
//   nch .. nch + 2NB - 1  the expanded V table (not copied): entry (step s, lane-entry
//                         L) is 4 tokens x fp16 at byte (s * 64 NB + L) * 8
// then the 1 KB dummy block.
//
// NB = 0 is the logits pass of a two-pass call (V ranks too wide for P @ V here): no V
// table and no P @ V; the softmax stores each valid logit (log2 domain, K scales
// applied, fp32) into the workspace logits buffer and keeps m and l for the partials.

#include <type_traits>

#include "decode_pages.hpp"

namespace starkv {

namespace {

// Dynamic LDS limit: 160 KB per CU minus the static arrays (partial and outlier-dot rows,
// P tables, alpha, outlier masks, head ids: under 20 KB).
constexpr int Q_MAX_DYN_LDS = 160 * 1024 - 20 * 1024;

// LDS address (buffer 0, relative to the page block) of byte b of row t.
__device__ __forceinline__ uint32_t row_byte(int b, int t) {
    return (uint32_t)((CS_CHUNKS + (b >> 6)) * PAGE_STRIDE + ((b >> 4) & 3) * 256 + 16 * t + (b & 15));
}

// Byte offset of V-table entry (step s, lane-entry L) from the table's first chunk.
__device__ __forceinline__ uint32_t vt_offset(int logical) {
    return (uint32_t)((logical >> 10) * PAGE_STRIDE + (logical & 1023));
}
template <int NB>
constexpr uint32_t vt_step_offset(int s, int nb) {  // entry (s, 64 nb) for lane 0
    return (uint32_t)(((s * NB + nb) >> 1) * PAGE_STRIDE + ((s * NB + nb) & 1) * 512);
}

// Per-lane LDS byte addresses (buffer 0), fixed for the whole kernel.
template <int MTV, int NB>
struct QLane {
    uint32_t cs[4];              // B operand: row lr, granule 4 ks + lg
    uint32_t k[MTV];             // slot i: the tile's 8 code bytes of row lr
    uint32_t st[(MTV + 3) / 4];  // partial-logit row of this lane's slot in each group of 4
    uint32_t sm;                 // softmax: first of the 4 rows of head lane >> 4
    uint32_t ksm;                // softmax: the (outlier, inlier) K scales of head lane >> 4, row lane & 15
    uint32_t so;                 // outlier-dot row of this lane's slot among kernel slots 0 .. 3
    uint32_t pw;                 // P * s_out write (head lane >> 4, token lane & 15); P * s_in at +128
    uint32_t vs;                 // the (outlier, inlier) V scales of row lane & 15
    uint32_t pa[NB > 0 ? NB : 1];  // P @ V A operand: P * s_out or P * s_in of head lane & 3
    uint32_t vt;                 // V table entry (0, lane)
    uint32_t cv_rd[NB > 0 ? NB : 1], cv_wr[NB > 0 ? NB : 1];  // V expansion: the byte read, the entry written
    int lg;                      // NB = 0: this lane's logit offset in a page's block (q head x 16 + token)
    uint32_t mk;                 // outlier masks of this lane's row group (table row 0)
    uint32_t sel;                // byte permute: bytes g, g + 4 -> bytes 0, 2
    uint32_t magic;              // 0x64006400
};

// Copy points of an iteration: 0 after the barrier and the V expansion, 1 .. MTV after
// each K tile, MTV + 1 after the softmax (the P @ V steps of the first page do not run,
// so they carry no copies).
template <int MTV>
struct QSched {
    static constexpr int NPOS = MTV + 2;
    static constexpr float time(int pos) {
        return pos == 0 ? 0.f : pos <= MTV ? 0.05f + 0.65f * (float)pos / (float)MTV : 0.95f;
    }
};

// (v & mask) | orv in one VOP3 instruction: the mask from an SGPR, orv from a VGPR (a
// VOP3 instruction on this target takes no literal and one scalar operand).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(orv));
    return r;
}

// a . b over two fp16 pairs with a zero accumulator (the inline constant, no register).
__device__ __forceinline__ float dot2_0(half2_t a, half2_t b) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// One tile's codes for this lane, decoded, with its z values in fp16: z holds ranks
// (2g, 2g+8, 2g+1, 2g+9), the last two scaled by 1/16; xa, xb their codes from the low
// and high nibbles of bytes g and g + 4 of w. magic = 0x64006400 (fp16 1024, both halves)
// held in a VGPR. d = the full dot.
struct QDec {
    half2_t xa, xb, za, zb;
    float d;
};

__device__ __forceinline__ QDec q_decode(const f32x4_t& z, uint2 w, uint32_t sel, uint32_t magic) {
    QDec t;
    const uint32_t v = __builtin_amdgcn_perm(w.y, w.x, sel);
    t.xa = as_h2(and_or(v, 0x000F000Fu, magic)) - (half2_t){(_Float16)1032.f, (_Float16)1032.f};
    t.xb = as_h2(and_or(v, 0x00F000F0u, magic)) - (half2_t){(_Float16)1152.f, (_Float16)1152.f};
    t.za = cvt_h2(z[0], z[1]);
    t.zb = cvt_h2(z[2], z[3]);
    t.d = dot2(t.xa, t.za, dot2_0(t.xb, t.zb));
    return t;
}

// The dot over the outlier ranks alone: the codes masked by m (fp16 halves).
__device__ __forceinline__ float q_outlier(const QDec& t, uint2 m) {
    return dot2(as_h2(h2_bits(t.xa) & m.x), t.za, dot2_0(as_h2(h2_bits(t.xb) & m.y), t.zb));
}

// Per-slot wave-uniform values packed into SGPR words (8 bits per slot, 4 per word) and
// re-read through an opaque SGPR, so they are not unpacked into SGPRs held across the
// loop: the tile of each kernel slot, the outlier ranks of its tile, its local head.
template <int MTV>
struct SlotPack {
    uint32_t tile[(MTV + 3) / 4], nout[(MTV + 3) / 4], head[(MTV + 3) / 4];
};
template <int MTV>
__device__ __forceinline__ int unpack8(const uint32_t (&w)[(MTV + 3) / 4], int i) {
    return (int)((uint32_t)opaque_s((int)w[i / 4]) >> (8 * (i % 4))) & 255;
}

// Kernel slots 0 .. 3 (the heads' first tiles) also compute the outlier dot; later
// slots do not, unless GEN: then every slot with outlier ranks adds its outlier dot to
// its head's row (heads with nout > 16).
constexpr int Q_OUTLIER_SLOTS = 4;
// Outlier-dot row of local head k in a wave's partial table: Q_EROW + 4 k, at a fixed
// distance from the head's first logit row 4 k (the softmax reads both off one address).
constexpr int Q_EROW = MAX_SLOTS + 1;
constexpr int Q_PART_ROWS = Q_EROW + 4 * 3 + 1;

// Adds this tile's outlier dot (summed over the row groups) to its head's row.
__device__ __forceinline__ void q_add_outlier(float e, uint32_t sp, int head, int lane) {
    const float r = sum_rows(e);
    const uint32_t a = sp + (uint32_t)((Q_EROW + 4 * head) * TILE_TOK + (lane & 15)) * 4;
    if (lane < 16) lds_st<float>(a, lds_ld<float>(a) + r);
}

// K side of one page (buffer B): MTV slots from VGPR AB, more from L2. Each group of 4
// slots is summed over the row groups with the lane swaps and stored as 4 rows.
// `hook(i)` runs after tile i's lane work (i a constant once the loop is unrolled): the
// iteration's other work rides under the tiles' MFMAs there.
template <bool GEN, int MTV, int NB, int B, int NLD, int BN, class Hook>
__device__ __forceinline__ void q_kside(const DecodeParams& p, const QLane<MTV, NB>& la, const half8_t (&ab)[MTV][4],
                                        const SlotPack<MTV>& sp8, int ntw, int nh, int nf, bool fast, uint32_t sp,
                                        uint32_t base, int lane, int wave, int cur_b, const DmaConst& dc,
                                        const DmaPage& dp, const uint32_t (&doff)[NLD], Hook&& hook) {
    half8_t csb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) csb[ks] = lds_ld<half8_t>(la.cs[ks] + B * 1024);
    float v[4], e[4];
    // Software pipelined: tile i + 1's MFMAs and code word are issued before tile i's
    // lane work, so they run under it.
    f32x4_t z = mfma_tile(ab[0], csb);
    uint2 w = lds_ld2(la.k[0] + B * 1024);
#pragma unroll
    for (int i = 0; i < MTV; ++i) {
        const f32x4_t zn = i + 1 < MTV ? mfma_tile(ab[i + 1 < MTV ? i + 1 : i], csb) : z;
        const uint2 wn = i + 1 < MTV ? lds_ld2(la.k[i + 1 < MTV ? i + 1 : i] + B * 1024) : w;
        const QDec t = q_decode(z, w, la.sel, la.magic);
        v[i & 3] = t.d;
        if (i < Q_OUTLIER_SLOTS) {
            e[i] = q_outlier(t, lds_ld2(la.mk + (uint32_t)unpack8<MTV>(sp8.nout, i) * 32u));
        } else if (GEN) {
            const int c = unpack8<MTV>(sp8.nout, i);
            if (c != 0) q_add_outlier(q_outlier(t, lds_ld2(la.mk + (uint32_t)c * 32u)), sp, unpack8<MTV>(sp8.head, i),
                                      lane);
        }
        z = zn;
        w = wn;
        hook(i);
        if ((i & 3) == 3 || i == MTV - 1) {
            const float r = sum_rows4(v[0], (i & 3) >= 1 ? v[1] : 0.f, (i & 3) >= 2 ? v[2] : 0.f,
                                      (i & 3) >= 3 ? v[3] : 0.f);
            lds_st<float>(la.st[i >> 2], r);
        }
        if (i == Q_OUTLIER_SLOTS - 1) {
            lds_st<float>(la.so, sum_rows4(e[0], e[1], e[2], e[3]));  // slots past nf: the spare row
            if (GEN) {
#pragma unroll
                for (int j = 0; j < Q_OUTLIER_SLOTS; ++j)
                    if (j >= nf && unpack8<MTV>(sp8.nout, j) != 0) q_add_outlier(e[j], sp, unpack8<MTV>(sp8.head, j), lane);
            }
        }
        copies_at<QSched<MTV>, NLD, BN>(1 + i, dc, dp, opaque_s(wave), doff);
    }
    if (ntw > MTV) {  // slots past MTV: AB from the workspace (L2) on every page
        const int lr = lane & 15;
        cint_p pw = (cint_p)(p.ws + p.ws_plan) + wave * PLAN_STRIDE;
        const half8_t* abg = (const half8_t*)(p.ws + p.ws_ab + (size_t)cur_b * p.TT * AB_TILE_BYTES);
        for (int i = MTV; i < ntw; ++i) {
            const uint32_t wd = (uint32_t)pw[PW_SLOTS + i];
            const int t = sw_tile(wd), c = sw_nout(wd);
            half8_t a[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) a[ks] = abg[(t * 4 + ks) * 64 + lane];
            const uint32_t ka = base + row_byte(8 * sw_code(wd), lr) + B * 1024;
            const QDec td = q_decode(mfma_tile(a, csb), lds_ld2(ka), la.sel, la.magic);
            const float r = sum_rows(td.d);
            if (lane < 16) lds_st<float>(sp + (uint32_t)(sw_row(wd) * TILE_TOK + lr) * 4, r);
            if (c != 0) q_add_outlier(q_outlier(td, lds_ld2(la.mk + (uint32_t)c * 32u)), sp, sw_head(wd), lane);
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): no tracked load left pending
    }
}

// Online softmax of the wave's heads (head lane >> 4 on a 16-lane row, token lane & 15)
// for the page in buffer B; writes P * s_out and P * s_in of the page's V scales.
// Returns true when some head's reference max moved (acc needs rescaling by alpha).
// ksw, vsw: this lane's (outlier, inlier) K scales of its head and V scales, row lane & 15.
template <int MTV, int NB>
__device__ __forceinline__ bool q_softmax(SmState& sm, const QLane<MTV, NB>& la, bool fast, uint32_t sp, int nh,
                                          uint32_t ksw, uint32_t vsw, uint32_t salpha, uint32_t shfn, int lane,
                                          int tok0, int lo, int hi, float* lgd = nullptr) {
    const uint32_t sm_addr = la.sm, pw_addr = la.pw;
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
    // The head's K scales for this token: s_in * (all ranks) + (s_out - s_in) * (outlier ranks).
    const float si = __uint_as_float(ksw & 0xffff0000u);
    s = fmaf(__uint_as_float(ksw << 16) - si, lds_ld<float>(sm_addr + Q_EROW * TILE_TOK * 4), si * s);
    const int tok = tok0 + lr;
    const bool valid = tok >= lo && tok < hi && kh < nh;
    s = valid ? s : -INFINITY;
    if (NB == 0 && valid) *lgd = s;
    float alpha = 1.f;
    bool moved = false;
    if (__builtin_amdgcn_ballot_w64(s > sm.m + LAZY_MAX) != 0) {
        const float mn = fmaxf(sm.m, row16_max(s));
        alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(sm.m - mn);
        sm.m = mn;
        moved = true;
        if (NB > 0 && lr == 0) lds_st<float>(salpha + 4 * (opaque(lane) >> 4), alpha);
    }
    const float pe = s == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - sm.m);
    sm.l = fmaf(sm.l, alpha, pe);
    if (NB == 0) return moved;
    lds_st<uint16_t>(pw_addr, __builtin_bit_cast(uint16_t, (_Float16)(pe * __uint_as_float(vsw << 16))));
    lds_st<uint16_t>(pw_addr + 128, __builtin_bit_cast(uint16_t, (_Float16)(pe * __uint_as_float(vsw & 0xffff0000u))));
    return moved;
}

// Expands the V nibbles of a page into the V table of buffer B: this thread's two
// lane-entries (the byte xv[k], read from the page) of one token per 64-lane block.
template <int NB, int B>
__device__ __forceinline__ void q_expand_v(const uint32_t (&xv)[NB], const uint32_t (&wr)[NB]) {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        const uint32_t byte = xv[k];
        const uint32_t x = (byte & 0xFu) | ((byte << 12) & 0xF0000u) | 0x64006400u;
        const uint32_t y = h2_bits(as_h2(x) - (half2_t){(_Float16)1032.f, (_Float16)1032.f});
        lds_st<uint16_t>(wr[k] + B * 1024, (uint16_t)y);
        lds_st<uint16_t>(wr[k] + B * 1024 + 8, (uint16_t)(y >> 16));
    }
}

// One step (4 tokens) of P @ V for the page whose V table is in buffer B: the operands
// are read one tile before the MFMA that uses them.
template <int NB>
struct PvStep {
    uint2 a[NB > 0 ? NB : 1], b[NB > 0 ? NB : 1];
};
template <int NB, int B>
__device__ __forceinline__ void pv_load(PvStep<NB>& q, const uint32_t (&pa)[NB > 0 ? NB : 1], uint32_t vt, int s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        q.a[nb] = lds_ld2(pa[nb] + 8 * s);
        q.b[nb] = lds_ld2(vt + vt_step_offset<NB>(s, nb) + B * 1024);
    }
}
template <int NB>
__device__ __forceinline__ void pv_mfma(f32x4_t (&acc)[NB > 0 ? NB : 1], const PvStep<NB>& q) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, q.a[nb]),
                                                     __builtin_bit_cast(half4_t, q.b[nb]), acc[nb], 0, 0, 0);
}

// acc[nb] = alpha * acc[nb] + (P * s)[4 heads, 16 tokens] @ V[16 tokens, lane-entries]
// for the page whose V table is in buffer B, on v_mfma_f32_4x4x4_16b with a per-block A.
template <int NB, int B>
__device__ __forceinline__ void q_pv(f32x4_t (&acc)[NB > 0 ? NB : 1], const uint32_t (&pa)[NB > 0 ? NB : 1],
                                     uint32_t vt, uint32_t salpha, bool rescale) {
    if (rescale) {
        const f32x4_t al = lds_ld<f32x4_t>(salpha);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[nb][e] *= al[e];
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint2 a = lds_ld2(pa[nb] + 8 * s);
            const uint2 b = lds_ld2(vt + vt_step_offset<NB>(s, nb) + B * 1024);
            acc[nb] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, a), __builtin_bit_cast(half4_t, b),
                                                         acc[nb], 0, 0, 0);
        }
    }
}

// The partial of a request: m, l and acc of this wave's heads into partial slot `slot`,
// then reset. colv[nb] = the V column of this lane's entry in block nb (-1: none).
template <int NB>
__device__ __forceinline__ void q_flush(const DecodeParams& p, SmState& sm, f32x4_t (&acc)[NB > 0 ? NB : 1], int nh,
                                        int slot, const int* sqh, int lane, const int (&colv)[NB > 0 ? NB : 1]) {
    const int ln = opaque(lane);
    const int kh = ln >> 4, lr = ln & 15;
    const int64_t base = (int64_t)slot * p.Hq;
    const float lt = row16_sum(sm.l);
    if (kh < nh && lr == 0) {
        const int qh = sqh[kh];
        ((float*)(p.ws + p.ws_m))[base + qh] = sm.m;
        ((float*)(p.ws + p.ws_l))[base + qh] = lt;
    }
    sm.m = -INFINITY;
    sm.l = 0.f;
    float* wa = (float*)(p.ws + p.ws_acc) + base * p.v_rank;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int qh = sqh[e];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (e < nh && colv[nb] >= 0) wa[(int64_t)qh * p.v_rank + colv[nb]] = acc[nb][e];
            acc[nb][e] = 0.f;
        }
    }
}

struct QLoop : PageLoop {
    bool pv;        // the previous page waits for its P @ V
    bool pv_moved;  // its softmax moved a reference max
    bool pv_end;    // it ended its request: flush after its P @ V
    int pv_b;       // its request
    int pv_buf;     // its buffer, when the loop ends
};

// One page of the loop: buffer BC holds page j (copied two pages ago), buffer BN
// receives page j + 2. Buffer BN held page j - 1: the copies do not touch its V table,
// which this iteration's P @ V reads.
template <bool GEN, int MTV, int NB, int NLD, int BC, int BN>
__device__ __forceinline__ bool q_iter(QLoop& st, const DmaConst& dc, const QLane<MTV, NB>& la,
                                       half8_t (&ab)[MTV][4], const SlotPack<MTV>& sp8,
                                       f32x4_t (&acc)[NB > 0 ? NB : 1], SmState& sm,
                                       const uint32_t (&doff)[NLD], int ntw, int nh, int nf, bool fast, uint32_t sp,
                                       uint32_t salpha, uint32_t shfn, uint32_t base, const int* sqh,
                                       const int (&colv)[NB > 0 ? NB : 1], int lane, int wave) {
    const DecodeParams& p = params();
    if (st.j >= st.end) {
        st.pv_buf = BN;  // the last page's buffer: its P @ V runs after the loop
        return false;
    }
    const int b = pr_b(st.rc.bits), k = st.rc.k, rows = pr_rows(st.rc.bits);
    if (page_starts_seg(st)) {
        // This request's AB into registers; slots past the wave's tiles load tile 0.
        const half8_t* abp = (const half8_t*)(p.ws + p.ws_ab + (size_t)b * p.TT * AB_TILE_BYTES);
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            const int t = unpack8<MTV>(sp8.tile, i);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ab[i][ks] = abp[(t * 4 + ks) * 64 + lane];
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    }
    SKV_WAIT_VM_LGKM0(NLD);  // only the copies of page j + 1 may still be in flight
    lds_barrier();           // page j is in LDS, page j - 1's V table is complete; page j - 1 is done
    const DmaPage dp = dma_setup(dc, st.r2, st.j + 2 < st.end);
    // The record of the page the next iteration copies: it arrives under the next wait.
    const PageRec next = st.j + 3 < st.end ? page_rec(p, st.j + 3) : st.rc;
    // Reads of page j for the V expansion and the softmax, issued first: they complete
    // under the K side. Page j - 1's P @ V (its P was 0 before the first page) runs
    // inside the K side: its rescale first, then one step per tile.
    uint32_t xv[NB > 0 ? NB : 1];
#pragma unroll
    for (int k = 0; k < NB; ++k) xv[k] = lds_ld<uint8_t>(la.cv_rd[k] + BC * 1024);
    const uint32_t ksw = lds_ld<uint32_t>(la.ksm + BC * 1024);
    const uint32_t vsw = NB > 0 ? lds_ld<uint32_t>(la.vs + BC * 1024) : 0u;
    if (NB > 0 && st.pv_moved) {
        const f32x4_t al = lds_ld<f32x4_t>(salpha);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[nb][e] *= al[e];
    }
    copies_at<QSched<MTV>, NLD, BN>(0, dc, dp, opaque_s(wave), doff);
    PvStep<NB> pq;
    auto hook = [&](int i) {
        if constexpr (NB > 0) {
            if (i == 0) q_expand_v<NB, BC>(xv, la.cv_wr);
            if (i >= 1 && i <= 4) pv_mfma<NB>(acc, pq);
            if (i <= 3) pv_load<NB, BN>(pq, la.pa, la.vt, i);
        }
    };
    q_kside<GEN, MTV, NB, BC, NLD, BN>(p, la, ab, sp8, ntw, nh, nf, fast, sp, base, lane, wave, b, dc, dp, doff,
                                       hook);
#pragma unroll
    for (int i = MTV; i <= 4; ++i) hook(i);  // the P @ V steps a short K side left
    if constexpr (NB > 0) {
        if (st.pv_end) q_flush<NB>(p, sm, acc, nh, st.pv_b + st.g, sqh, lane, colv);
        st.pv_moved = q_softmax<MTV, NB>(sm, la, fast, sp, nh, ksw, vsw, salpha, shfn, lane, 0, 0, rows);
    } else {
        // The logits pass: page j's logits into the request's rows.
        float* lgd = (float*)(p.ws + p.ws_lg) + ((int64_t)b * (p.lcap / TILE_TOK) + k) * p.Hq * TILE_TOK + la.lg;
        q_softmax<MTV, NB>(sm, la, fast, sp, nh, ksw, vsw, salpha, shfn, lane, 0, 0, rows, lgd);
    }
    copies_at<QSched<MTV>, NLD, BN>(MTV + 1, dc, dp, opaque_s(wave), doff);
    const bool seg_end = page_ends_seg(st);
    if constexpr (NB == 0) {  // the request's partial (m, l) as soon as its last page is done
        if (seg_end) flush_partial<0>(p, sm, acc, nh, b + st.g, sqh, lane);
    }
    st.pv = true;
    st.pv_end = seg_end;
    st.pv_b = b;
    page_loop_next<3>(st, next);
    return true;
}

template <int MTV, int NB, int NLD>
__global__ __launch_bounds__(NTHR) void quant_kernel(const DecodeParams p0) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_pages[];
    __shared__ __attribute__((aligned(16))) float s_part[NWAVE][Q_PART_ROWS * TILE_TOK];
    __shared__ __attribute__((aligned(16))) uint16_t s_pq[NWAVE][2][4 * TILE_TOK];  // P * s_out, P * s_in
    __shared__ __attribute__((aligned(16))) float s_alpha[NWAVE][4];
    __shared__ __attribute__((aligned(16))) uint2 s_omask[17][4];  // [outlier ranks of the tile][row group]
    __shared__ int s_qh[NWAVE][4];
    __shared__ int s_hfn[NWAVE][4];  // per local head: first slot | slots << 8

    const DecodeParams& p = params();
    const int tid = threadIdx.x, lane = tid & 63, wave = rfl(tid >> 6);
    const int lg = lane >> 4, lr = lane & 15;
    cint_p plan = (cint_p)(p.ws + p.ws_plan);
    // Page buffers and partial-logit rows start zeroed: rows past a request's end are
    // never copied and must hold finite values (P is 0 there); a head's partial rows
    // past its slots are summed as zeros. Done first: it overlaps the header loads.
    for (int i = tid; i < p.lds_bytes / 16; i += NTHR) ((uint4*)s_pages)[i] = make_uint4(0, 0, 0, 0);
    for (int i = tid; i < NWAVE * Q_PART_ROWS * TILE_TOK; i += NTHR) (&s_part[0][0])[i] = 0.f;
    if (tid < NWAVE * 4) (&s_alpha[0][0])[tid] = 1.f;
    for (int i = tid; i < NWAVE * 2 * 4 * TILE_TOK; i += NTHR) (&s_pq[0][0][0])[i] = 0;  // P before the first page
    if (tid < 17 * 4) {  // fp16-half masks of the outlier ranks among (2g, 2g+8 | 2g+1, 2g+9) for c outliers
        const int c = tid >> 2, g = tid & 3;
        const uint32_t ma = (2 * g < c ? 0x0000ffffu : 0u) | (2 * g + 8 < c ? 0xffff0000u : 0u);
        const uint32_t mb = (2 * g + 1 < c ? 0x0000ffffu : 0u) | (2 * g + 9 < c ? 0xffff0000u : 0u);
        s_omask[c][g] = make_uint2(ma, mb);
    }
    // The logits pass of a step whose direct write left its V latents to pack: the last
    // wave of each workgroup packs the workgroup's share of their bytes (P @ V, the next
    // launch, reads them); its loads are issued here and used after the setup below.
    const bool vpk = NB == 0 && wave == NWAVE - 1 && p.vp.n > 0;
    const int vj0 = (int)((int64_t)blockIdx.x * p.vp.v_bytes / gridDim.x);
    const int vj1 = (int)((int64_t)(blockIdx.x + 1) * p.vp.v_bytes / gridDim.x);
    VPackPre vpre;
    if constexpr (NB == 0) {
        if (vpk && vpack_two_step(p.vp, vj0, vj1)) vpre = vpack_load(p.vp, vj0, vj1, lane);
    }
    auto vpack_share = [&]() {
        if constexpr (NB == 0) {
            if (vpk) {
                if (vpack_two_step(p.vp, vj0, vj1)) vpack_store(p.vp, vpre, vj0, vj1, blockIdx.x == 0, lane);
                else for (int t = 0; t < p.vp.n; ++t) vpack_range(p.vp, t, vj0, vj1, blockIdx.x == 0, lane);
            }
        }
    };
    QLoop st;
    const int planned = plan[NWAVE * PLAN_STRIDE], hS = ((cint_p)p.ws)[0], htot = ((cint_p)p.ws)[1 + p.n];
    __syncthreads();  // the zero fill is done on every wave before a page copy lands
    // No wave plan (the merge reports NaN) or no pages: the workgroup packs its share and leaves.
    if (planned == 0 || !page_loop_init<3>(st, p, xcd_range(blockIdx.x, gridDim.x), hS, htot)) {
        vpack_share();
        return;
    }
    // The first two pages' copies go out as soon as their records are in: the rest of the
    // setup (the wave plan, the lane addresses) runs under their latency.
    const uint32_t base = lds_addr(s_pages);
    uint32_t doff[NLD];  // copy offsets of this lane inside a page, per copy i (chunk 8 i + wave)
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ch = i * NWAVE + wave;
        uint32_t off = 0x80000000u;  // past the descriptor range: no memory access
        if (ch < CS_CHUNKS) {
            off = cs_copy_offset(ch, lane, p.cs_s0b);
        } else if (ch < p.nch) {
            const int G = 4 * (ch - CS_CHUNKS) + (lane >> 4), t = lane & 15;
            if (G < p.row_g) off = (uint32_t)(t * (int)p.c_s1 + 16 * G);
        }
        doff[i] = off;
    }
    const DmaConst dc = dma_const(p, base, wave, base + (uint32_t)((p.nch + 2 * NB) * PAGE_STRIDE));
    dma_page<NLD, 0>(dc, st.rc, true, wave, doff);
    dma_page<NLD, 1>(dc, st.r1, st.beg + 1 < st.end, wave, doff);

    // This wave's plan: slots (rank tiles) and heads (at most 4: Hq <= 32).
    cint_p pw = plan + wave * PLAN_STRIDE;
    const int ntw = pw[0], nh = pw[1];
    const bool fast = pw[3] != 0;
    const uint32_t sp = lds_addr(&s_part[wave][0]);
    const int O4 = (p.v_nout + 3) & ~3;
    const uint32_t vt0 = base + (uint32_t)(p.nch * PAGE_STRIDE);  // V table
    QLane<MTV, NB> la;
    SlotPack<MTV> sp8;
    bool gen = false;         // some kernel slot other than a head's first tile holds outlier ranks
    const int nf = pw[2];     // heads with tiles: kernel slots 0 .. nf - 1 are their first tiles
    uint32_t swd[MTV];        // the wave's slot words, in this kernel's order
#pragma unroll
    for (int i = 0; i < MTV; ++i) swd[i] = (uint32_t)pw[PW_SLOTS + i];
    {
#pragma unroll
        for (int w = 0; w < (MTV + 3) / 4; ++w) sp8.tile[w] = sp8.nout[w] = sp8.head[w] = 0;
#pragma unroll
        for (int i = 0; i < MTV; ++i) {
            la.k[i] = vgpr_pin(base + row_byte(8 * sw_code(swd[i]), lr));
            const int c = sw_nout(swd[i]);
            sp8.tile[i / 4] |= (uint32_t)sw_tile(swd[i]) << (8 * (i % 4));
            sp8.nout[i / 4] |= (uint32_t)c << (8 * (i % 4));
            sp8.head[i / 4] |= (uint32_t)sw_head(swd[i]) << (8 * (i % 4));
            gen = gen || (i >= nf && c > 0);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) la.cs[ks] = base + cs_read_offset(ks, lg, lr);
        const int rslot = ((lg & 1) << 1) | (lg >> 1);  // sum_rows4 puts inputs (a, b, c, d) in rows (0, 2, 1, 3)
#pragma unroll
        for (int g = 0; g < (MTV + 3) / 4; ++g) {
            int row = MAX_SLOTS;  // the row of kernel slot 4 g + rslot (past MTV: the spare row)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * g + j < MTV && rslot == j) row = sw_row(swd[4 * g + j < MTV ? 4 * g + j : 0]);
            la.st[g] = sp + (uint32_t)(row * TILE_TOK + lr) * 4;
        }
        la.sm = sp + (uint32_t)(4 * lg * TILE_TOK + lr) * 4;
        la.ksm = base + row_byte(p.ks_off + 4 * (lg < nh ? pw[32 + lg] : 0), lr);
        {  // the outlier-dot row of kernel slot rslot (0 .. 3): its tile's head
            int hk = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (rslot == j) hk = sw_head(swd[j]);
            la.so = sp + (uint32_t)(((rslot < nf ? Q_EROW + 4 * hk : MAX_SLOTS)) * TILE_TOK + lr) * 4;
        }
        la.pw = lds_addr(&s_pq[wave][0][0]) + (uint32_t)(lg * TILE_TOK + lr) * 2;
        la.vs = base + row_byte(p.vs_off, lr);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            la.pa[nb] = lds_addr(&s_pq[wave][64 * nb + lane < O4 ? 0 : 1][0]) + (uint32_t)(lane & 3) * TILE_TOK * 2;
        la.vt = vt0 + 8 * lane;
        la.lg = (lg < nh ? pw[32 + lg] : 0) * TILE_TOK + lr;
        // V expansion: token t = tid % 16, lane-entries L, L + 1 with L = 2 (tid / 16) + 64 k.
        const int t = tid & 15;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int L = 2 * (tid >> 4) + 64 * k;
            int b = p.vq_off;  // entries with no column read a valid byte and are never stored
            if (L < O4) {
                if (L < p.v_nout) b = p.vq_off + (L >> 1);
            } else if (p.v_nout + L - O4 < p.v_rank) {
                b = p.vq_off + p.v_nbo + ((L - O4) >> 1);
            }
            la.cv_rd[k] = base + row_byte(b, t);
            la.cv_wr[k] = vt0 + vt_offset((((t >> 2) * 64 * NB + L) << 3) + (t & 3) * 2);
        }
        la.mk = vgpr_pin(lds_addr(&s_omask[0][lg]));
        la.sel = vgpr_pin((uint32_t)lg | 0x0c00u | ((uint32_t)(4 + lg) << 16) | 0x0c000000u);
        la.magic = vgpr_pin(0x64006400u);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) la.cs[ks] = vgpr_pin(la.cs[ks]);
        la.sm = vgpr_pin(la.sm);
        la.ksm = vgpr_pin(la.ksm);
        la.so = vgpr_pin(la.so);
        la.pw = vgpr_pin(la.pw);
        la.vs = vgpr_pin(la.vs);
        la.vt = vgpr_pin(la.vt);
#pragma unroll
        for (int g = 0; g < (MTV + 3) / 4; ++g) la.st[g] = vgpr_pin(la.st[g]);
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            la.pa[k] = vgpr_pin(la.pa[k]);
            la.cv_rd[k] = vgpr_pin(la.cv_rd[k]);
            la.cv_wr[k] = vgpr_pin(la.cv_wr[k]);
        }
    }
    int colv[NB > 0 ? NB : 1];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int L = 64 * nb + lane;
        colv[nb] = L < O4 ? (L < p.v_nout ? L : -1) : (p.v_nout + L - O4 < p.v_rank ? p.v_nout + L - O4 : -1);
    }
    const uint32_t salpha = lds_addr(&s_alpha[wave][0]);
    if (lane < 4) s_qh[wave][lane] = lane < nh ? pw[32 + lane] : 0;
    SmState sm;
    if (lane < 4) s_hfn[wave][lane] = lane < nh ? pw[40 + lane] | (pw[48 + lane] << 8) : 0;
    const uint32_t shfn = lds_addr(&s_hfn[wave][0]);
    sm.m = -INFINITY;
    sm.l = 0.f;

    vpack_share();
    __syncthreads();

    st.pv = false;
    st.pv_moved = false;
    st.pv_end = false;
    st.pv_b = 0;
    st.pv_buf = 0;

    half8_t ab[MTV][4];
    f32x4_t acc[NB > 0 ? NB : 1];
#pragma unroll
    for (int k = 0; k < (NB > 0 ? NB : 1); ++k) acc[k] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    const int* sqh = &s_qh[wave][0];
    // The page loop, in one of two forms picked per wave (see q_kside).
    auto loop = [&](auto gen_tag) {
        constexpr bool G = decltype(gen_tag)::value;
        while (true) {
            if (!q_iter<G, MTV, NB, NLD, 0, 2>(st, dc, la, ab, sp8, acc, sm, doff, ntw, nh, nf, fast, sp, salpha, shfn, base, sqh,
                                               colv, lane, wave))
                break;
            if (!q_iter<G, MTV, NB, NLD, 1, 0>(st, dc, la, ab, sp8, acc, sm, doff, ntw, nh, nf, fast, sp, salpha, shfn, base, sqh,
                                               colv, lane, wave))
                break;
            if (!q_iter<G, MTV, NB, NLD, 2, 1>(st, dc, la, ab, sp8, acc, sm, doff, ntw, nh, nf, fast, sp, salpha, shfn, base, sqh,
                                               colv, lane, wave))
                break;
        }
    };
    if (gen)
        loop(std::true_type{});
    else
        loop(std::false_type{});
    // The last page's P @ V, once its V table is visible to every wave.
    SKV_WAIT_VM_LGKM0(0);  // also: no copy may land after the workgroup ends
    lds_barrier();
    if (NB > 0 && st.pv) {
        q_pv<NB, 0>(acc, la.pa, la.vt + (uint32_t)st.pv_buf * 1024u, salpha, st.pv_moved);
        q_flush<NB>(p, sm, acc, nh, st.pv_b + st.g, sqh, lane, colv);
    }
}

// The instantiations that run without scratch spills (MTV tiles per wave in VGPRs, NB V
// blocks, NLD copies per wave). Only these are compiled (quant_mtv picks among them).
constexpr bool q_spill_free(int mtv, int nb, int nld) {
    return mtv <= 4 || (mtv <= 8 && nb <= 3) || (mtv == 9 && nb <= (nld <= 3 ? 2 : 1)) ||
           (mtv == 10 && nb <= (nld <= 3 ? 1 : 0));
}

template <int MTV, int NB, int NLD>
const void* q_inst() {
    if constexpr (q_spill_free(MTV, NB, NLD)) return (const void*)&quant_kernel<MTV, NB, NLD>;
    return nullptr;
}

template <int MTV, int NLD>
const void* q_pick_nb(int nb) {
    if (nb <= 0) return q_inst<MTV, 0, NLD>();
    if (nb <= 1) return q_inst<MTV, 1, NLD>();
    if (nb <= 2) return q_inst<MTV, 2, NLD>();
    if (nb <= 3) return q_inst<MTV, 3, NLD>();
    return q_inst<MTV, 5, NLD>();
}

template <int NLD>
const void* q_pick_mtv(int mtv, int nb) {
    return mtv == 4 ? q_pick_nb<4, NLD>(nb)
           : mtv == 8 ? q_pick_nb<8, NLD>(nb)
           : mtv == 9 ? q_pick_nb<9, NLD>(nb)
                      : q_pick_nb<10, NLD>(nb);
}

int q_nb_blocks(int nb) { return nb <= 0 ? 0 : nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 3 ? 3 : 5; }

}  // namespace

// 64-lane P @ V blocks of the 3.2-bit kernel: the outlier columns padded to 4, then the
// inlier columns (0 if more than 5 blocks are needed).
int quant_v_blocks(int v_rank, int v_nout) {
    const int lanes = ((v_nout + 3) & ~3) + (v_rank - v_nout);
    const int nb = (lanes + 63) / 64;
    return nb <= 5 ? q_nb_blocks(nb) : 0;
}

int quant_chunks(int row_bytes) { return CS_CHUNKS + (row_bytes / 16 + 3) / 4; }

int quant_copies(int row_bytes) {
    const int nld = (quant_chunks(row_bytes) + NWAVE - 1) / NWAVE;
    return nld <= 3 ? 3 : nld <= 6 ? 6 : 0;
}

int quant_lds_bytes(int row_bytes, int nb) { return (quant_chunks(row_bytes) + 2 * nb) * PAGE_STRIDE + 1024; }

int quant_lds_limit() { return Q_MAX_DYN_LDS; }

// Rank tiles per wave held in VGPRs (as lowrank_mtv): the smallest compiled size >= need,
// or the next smaller one if that one would spill and it still holds need - 1; 0 if
// neither runs without spills with nb V blocks (the two-pass form then).
int quant_mtv(int TT, int nb, int row_bytes) {
    static const int sizes[4] = {4, 8, 9, 10};
    const int need = (TT + NWAVE - 1) / NWAVE, nld = quant_copies(row_bytes), nbv = q_nb_blocks(nb);
    int i = 0;
    while (i < 3 && sizes[i] < need) ++i;
    if (q_spill_free(sizes[i], nbv, nld)) return sizes[i];
    if (i > 0 && sizes[i - 1] >= need - 1 && q_spill_free(sizes[i - 1], nbv, nld)) return sizes[i - 1];
    return 0;
}

int launch_quant(const DecodeParams& p, int nb, int grid, hipStream_t stream) {
    const int mtv = quant_mtv(p.TT, nb, p.row_g * 16);
    const int nld = quant_copies(p.row_g * 16);
    SKV_CHECK(mtv > 0, "decode: no spill-free kernel for %d rank tiles and %d V blocks", p.TT, nb);
    const void* fn = nld <= 3 ? q_pick_mtv<3>(mtv, nb) : q_pick_mtv<6>(mtv, nb);
    SKV_CHECK(fn != nullptr, "decode: no kernel for %d rank tiles and %d V blocks", p.TT, nb);
    static const void* raised[256];  // kernels whose dynamic-LDS limit was raised (host-side bookkeeping)
    static int nraised = 0;
    bool seen = false;
    for (int i = 0; i < nraised; ++i) seen = seen || raised[i] == fn;
    if (!seen) {
        SKV_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, Q_MAX_DYN_LDS));
        if (nraised < 256) raised[nraised++] = fn;
    }
    void* args[] = {(void*)&p};
    SKV_HIP(hipLaunchKernel(fn, dim3(grid), dim3(NTHR), args, (size_t)p.lds_bytes, stream));
    return STARKV_OK;
}

}  // namespace starkv
