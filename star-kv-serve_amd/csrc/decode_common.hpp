// Shared definitions of the paged decode launches (decode.hip, decode_lowrank.hip,
// decode_quant.hip):
// constants, the workspace layout and page records, the kernel parameter block, the
// global->LDS copy primitive and the per-partial flush.
#pragma once

#include <stdio.h>

#include <algorithm>

#include "common.hpp"
#include "pack_rows.hpp"

namespace starkv {
enum { FMT_BF16 = 0, FMT_F16 = 1, FMT_Q4 = 2 };

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

constexpr int NWAVE = 8;
constexpr int NTHR = NWAVE * 64;
constexpr int TILE_TOK = 16;
constexpr int MAX_REQ_PER_CALL = 1024;
constexpr float LOG2E = 1.4426950408889634f;
constexpr int AB_TILE_BYTES = 4 * 64 * 16;  // 4 K-steps x 64 lanes x 8 fp16
constexpr int AB_SLACK_TILES = 16;
constexpr int MAX_TT = 96;                  // rank tiles per call (k_width x heads per kv head <= 1536)
constexpr int MAX_H = 32;                   // query heads
constexpr int MAX_HW = 8;                   // query heads per wave
constexpr int MAX_SLOTS = 16;               // rank tiles per wave
constexpr int PLAN_STRIDE = 80;             // ints per wave in the plan
constexpr int PW_SLOTS = 64;                // first slot word in a wave's plan
constexpr int CS_ROW_LDS = 256;             // LDS bytes per cos/sin row (granules XOR-swizzled by row)
constexpr int CS_CHUNKS = 4;                // 16 rows x 16 granules -> 4 copies of 64 granules
constexpr float LAZY_MAX = 8.f;             // log2 headroom before the running max moves

// Workspace layout, in bytes from the base (every region 256-byte aligned):
//   hdr    int   [2 + n]      S (pages per decode workgroup), P[0..n] (prefix of the
//                             requests' page counts ceil(min(len, max_seq_len) / 16))
//   pages  PageRec [n * ceil(max_seq_len / 16)]  one record per page, request after
//                             request (page P[b] + k is page k of request b)
//   plan   int   [8][80] + 1  per wave: [0] tiles, [1] heads, [2] heads with tiles,
//                             [3] 1 if every head has <= 4 tiles, [8 + s] tile of slot s,
//                             [32 + k] q head of local head k, [40 + k] its first slot,
//                             [48 + k] its slots, [64 + i] slot word of the decode kernel's
//                             slot i (below); then 1 if every head found a wave
//   ab     fp16  [n][TT][4][64][8]
//   m, l   fp32  [slots][Hq]  (log2-domain reference max and sum per partial)
//   acc    fp32  [slots][Hq][v_rank]
//   lg     fp32  [n][lcap/16][Hq][16]  (two-pass calls only) log2-domain logits, page
//                               major: token l of request b, head h at
//                               ((b lcap/16 + l/16) Hq + h) 16 + l % 16 (a page's logits of
//                               every head are one 2 KB block), lcap = max_seq_len
//                               rounded up to 16
//   o      fp32  [n][Hq][ld]    (two-pass calls only) merged low-rank outputs
// Two-pass calls pad acc and o rows to ld = v_rank rounded up to 4 (16-byte rows). Their
// P @ V pass runs over ranges of R consecutive logits-pass ranges (R >= 1, for few
// requests: the logits pass then spreads over more workgroups than the P @ V pass, whose
// partials are wide): pv slots = ceil(grid / R) + n, the acc rows are per pv slot, and m
// and l hold R ceil(grid / R) + n slots (the ranges past grid are never written).
// Slot word: everything a decode kernel needs of one of its slots, so that its prologue
// reads a wave's slots with a few wide scalar loads: the code tile (first cache lane /
// 16), the tile's outlier ranks (3.2-bit), the slot's partial-logit row, its local head
// and its tile. The row: with every head of the wave at <= 4 slots, head k's j-th slot
// goes to row 4 k + j, so a head's rows past its slots stay zero and the softmax sums 4
// fixed rows; otherwise the slot's place in the plan. Slots past the wave's tiles hold
// tile 0 and the spare row MAX_SLOTS.
constexpr uint32_t SW_CODE_MASK = 0x1FFF;  // bits 0-12: code tile; 13-17: outlier ranks
__host__ __device__ constexpr uint32_t slot_word(uint32_t code_nout, int row, int head, int tile) {
    return code_nout | ((uint32_t)row << 18) | ((uint32_t)head << 23) | ((uint32_t)tile << 25);
}
__device__ __forceinline__ int sw_code(uint32_t w) { return (int)(w & SW_CODE_MASK); }
__device__ __forceinline__ int sw_nout(uint32_t w) { return (int)((w >> 13) & 31); }
__device__ __forceinline__ int sw_row(uint32_t w) { return (int)((w >> 18) & 31); }
__device__ __forceinline__ int sw_head(uint32_t w) { return (int)((w >> 23) & 3); }
__device__ __forceinline__ int sw_tile(uint32_t w) { return (int)(w >> 25); }

struct WsLayout {
    size_t hdr, pages, plan, ab, m, l, acc, lg, o, total;
    int ld;  // floats per acc / o row
};

static inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Page record: where a page's rows are and what the decode needs to know of it. The
// decode launches split the pages (not the tokens) into equal contiguous ranges, one per
// workgroup, and read one record per page with a scalar load: no token cursor, block
// table lookup or address arithmetic beyond one 64-bit add in the page loop.
//   addr  byte address of the page's first row (cache + block * c_s0 + slot * c_s1)
//   k     page index inside the request (its tokens are 16 k .. 16 k + rows - 1)
//   bits  request b (bits 0-10) | rows - 1 (bits 11-14) | 1 << 15 if the page is the
//         request's last
struct PageRec {
    uint64_t addr;
    int k;
    uint32_t bits;
};
constexpr uint32_t PR_LAST = 1u << 15;
__host__ __device__ constexpr uint32_t pr_bits(int b, int rows, bool last) {
    return (uint32_t)b | ((uint32_t)(rows - 1) << 11) | (last ? PR_LAST : 0u);
}
__device__ __forceinline__ int pr_b(uint32_t bits) { return (int)(bits & 0x7FF); }
__device__ __forceinline__ int pr_rows(uint32_t bits) { return (int)((bits >> 11) & 15) + 1; }
static inline int pages_of(int max_seq_len) { return (max_seq_len + 15) / 16; }

// lcap = 0: the one-pass decode (no logits buffer). pv_r: the P @ V pass's R. maxp: page
// records per request (pages_of(max_seq_len)).
static WsLayout ws_layout(int n, int Hq, int TT, int v_rank, int grid, int lcap, int pv_r, int maxp) {
    WsLayout w;
    const size_t gp = lcap > 0 ? ((size_t)grid + pv_r - 1) / pv_r : (size_t)grid;
    const size_t slots = (lcap > 0 ? std::max((size_t)grid, gp * pv_r) : (size_t)grid) + n;
    const size_t pslots = gp + n;
    size_t o = 0;
    w.hdr = o; o = al256(o + (size_t)(n + 2) * 4);
    w.pages = o; o = al256(o + (size_t)n * (size_t)maxp * sizeof(PageRec));
    w.plan = o; o = al256(o + (size_t)(NWAVE * PLAN_STRIDE + 1) * 4);
    w.ab = o; o = al256(o + ((size_t)n * TT + AB_SLACK_TILES) * AB_TILE_BYTES);
    w.m = o; o = al256(o + slots * Hq * 4);
    w.l = o; o = al256(o + slots * Hq * 4);
    w.ld = lcap > 0 ? (v_rank + 3) & ~3 : v_rank;
    w.acc = o; o = al256(o + pslots * Hq * (size_t)w.ld * 4);
    w.lg = o; o = al256(o + (size_t)n * Hq * (size_t)lcap * 4);
    w.o = o; o = al256(o + (lcap > 0 ? (size_t)n * Hq * (size_t)w.ld * 4 : 0));
    w.total = o;
    return w;
}

struct DecodeParams {
    const uint8_t* cache; int64_t c_s0, c_s1;      // bytes
    int bs_shift;                                  // block_size = 16 << bs_shift
    const int32_t* bt; int bt_s0, bt_s1;
    int n, Hq, TT, k_width, v_rank;
    int v_col;                                     // bf16/fp16: first V lane of a row (from the cache pointer)
    int ks_off, vs_off, vq_off, v_nout, v_nbo;     // QuantRow (3.2-bit)
    int row_g;                                     // row granules (16 B)
    int nch, lds_bytes;                            // 1 KB chunks copied per page, dynamic LDS bytes
    const uint8_t* cs; int cs_s0b;                 // fp16 cos/sin table, row stride in bytes
    uint8_t* ws;
    size_t ws_plan, ws_ab, ws_m, ws_l, ws_acc;
    size_t ws_lg; int lcap;                        // two-pass calls: logits buffer, row length
    size_t ws_o; int acc_ld;                       // two-pass calls: merged outputs; acc / o row floats
    int pv_r;                                      // two-pass calls: logits-pass ranges per P @ V range
    size_t ws_pages;                               // page records
    VPackParams vp;                                // 3.2-bit logits pass: a direct write's V latents (vp.n > 0)
};

__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int lds_ld_i32(uint32_t a) { return *(const __attribute__((address_space(3))) int*)(a); }

typedef const __attribute__((address_space(4))) int32_t* cint_p;

// ---------------------------------------------------------------------------
// Global -> LDS copies: raw buffer loads with the LDS bit, 16 bytes per lane.
// ---------------------------------------------------------------------------
typedef int int4v_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor: 48-bit base, stride 0, `bytes` in range (offsets at or past it
// are not read), gfx9 data format word.
__device__ __forceinline__ int4v_t buffer_rsrc(const void* base, int bytes) {
    const uint64_t a = (uint64_t)base;
    return (int4v_t){(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), bytes, 0x00020000};
}

// One 16-byte-per-lane global->LDS copy: lane q's 16 bytes at `voff` land at LDS
// byte lds + 16 q. Issued as inline assembly so that the compiler does not track it:
// it would otherwise wait for copies into other page buffers before reads of the
// current one. The waits for these copies are explicit (vmcnt at the page barrier).
// M0 takes the LDS address; one wait state separates the M0 write from its use.
__device__ __forceinline__ void lds_copy16(const int4v_t& rsrc, uint32_t lds, uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds), "v"(voff), "s"(rsrc)
        : "memory", "m0");
}

// The kernel's parameter block, read through a pointer the optimizer cannot see
// through: loads of it are redone where they are used (scalar loads that hit the
// scalar cache) instead of being hoisted out of the main loop into SGPRs.
typedef const __attribute__((address_space(4))) DecodeParams kparams_t;

__device__ __forceinline__ const DecodeParams& params() {
    kparams_t* pp = (kparams_t*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(pp));
    return *(const DecodeParams*)pp;  // address-space inference keeps these scalar loads
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t cvt_h2(float a, float b) {
    return __builtin_convertvector((float2_t){a, b}, half2_t);  // v_cvt_pk_f16_f32, round to nearest even
}
__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

__device__ __forceinline__ uint2 ld64(const uint8_t* p) {
    const uint64_t v = *(const uint64_t*)p;
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

__device__ __forceinline__ f32x4_t mfma_tile(const half8_t (&a)[4], const half8_t (&cs)[4]) {
    f32x4_t z = {0.f, 0.f, 0.f, 0.f};
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], cs[0], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], cs[1], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2], cs[2], z, 0, 0, 0);
    z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[3], cs[3], z, 0, 0, 0);
    return z;
}

// Online softmax of this wave's heads: local head (lane >> 4) on a 16-lane row, token
// lane & 15.
struct SmState {
    float m, l;   // log2-domain reference max (same on the head's 16 lanes), this lane's column sum
};

// A wave's heads' partial-logit rows for the softmax of heads with more than 4 slots (the
// rare path): per local head k, its first slot | its slots << 8, kept in LDS rather than
// registers (the common path never reads them).
__device__ __forceinline__ int head_slots(uint32_t shfn, int lane) { return lds_ld_i32(shfn + 4 * (opaque(lane) >> 4)); }

// The partial of the request that ends with this page: m, l and acc of this wave's
// heads into partial slot `slot`, then reset. The wave's query-head ids come from LDS:
// a vector load here would leave a tracked load in flight at the loop's join, and the
// compiler would then drain every copy before the next page's first LDS read.
// NB = 0 (the logits pass of a two-pass call): m and l only.
template <int NB>
__device__ __forceinline__ void flush_partial(const DecodeParams& p, SmState& sm, f32x4_t (&acc)[NB > 0 ? NB : 1],
                                              int nh, int slot, const int* sqh, int lane) {
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
            const int c = 64 * nb + ln;
            if (e < nh && c < p.v_rank) wa[(int64_t)qh * p.v_rank + c] = acc[nb][e];
            acc[nb][e] = 0.f;
        }
    }
}

// The bf16/fp16 decode kernel (decode_lowrank.hip): picks the instantiation for
// (fmt, v column blocks nb, rank tiles per wave) and launches it on `stream`.
int launch_lowrank(const DecodeParams& p, int fmt, int nb, int grid, hipStream_t stream);
// The bf16/fp16 kernel's page geometry for (k_width, V column blocks nb): 1 KB chunks
// per page, page buffers (3 or 2), dynamic LDS bytes, copies per wave per page (0 if a
// page does not fit).
int lowrank_chunks(int k_width, int nb);
// Rank tiles per wave the bf16/fp16 kernel holds in VGPRs for TT rank tiles and nb V
// blocks (nb = 0: the logits pass); 0 if no instantiation runs the one pass without
// scratch spills.
int lowrank_mtv(int TT, int nb);
int lowrank_buffers(int k_width, int nb);
int lowrank_lds_bytes(int k_width, int nb);
int lowrank_copies(int k_width, int nb);

// The 3.2-bit decode kernel (decode_quant.hip) and its page geometry: P @ V blocks for
// (v_rank, v_nout) (0 if too many), 1 KB chunks copied per page and copies per wave (0 if
// a page does not fit) for a row of row_bytes, dynamic LDS bytes, the LDS limit.
int launch_quant(const DecodeParams& p, int nb, int grid, hipStream_t stream);

// The two-pass decode (decode_wide.hip): the P @ V pass over the logits the K pass
// stored (one launch per column window), whether its pages fit in LDS, and the merge of
// its partials with the lift through v_up_by_q (of dtype w_dt).
// Compute units of the current device (cached per device).
int device_cus();
int launch_pv(const DecodeParams& p, int fmt, int grid, hipStream_t stream);
bool pv_fits(int fmt, int k_width, int v_rank, int vs_off, int vq_off, int v_nout, int v_bytes);
int launch_merge_wide(const DecodeParams& p, int grid, int w_dt, const void* vup, int64_t vu_s0, int64_t vu_s1,
                      void* out, int64_t o_s0, int64_t o_s1, int out_dt, hipStream_t stream);
constexpr int MAX_V_RANK_TWO_PASS = 4096;  // H x head_dim of a 32-head MHA layer: a full-rank V
int quant_v_blocks(int v_rank, int v_nout);
int quant_mtv(int TT, int nb, int row_bytes);  // as lowrank_mtv, for the 3.2-bit kernel
int quant_chunks(int row_bytes);
int quant_copies(int row_bytes);
int quant_lds_bytes(int row_bytes, int nb);
int quant_lds_limit();

}  // namespace starkv
