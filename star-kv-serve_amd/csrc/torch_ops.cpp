// torch.ops.starkv: the PyTorch-ROCm operator layer over the C ABI (libstarkv_hip.so).
//
// Each operator takes tensors, reads their pointers, strides and dtypes, allocates the
// call's workspace from torch's caching allocator on the current stream, launches on the
// current HIP stream of the tensors' device and turns a library error into a
// c10::Error carrying the library's message. Registered for the CUDA (ROCm) dispatch
// key only: a CPU tensor has no kernel here and raises. The Python wrappers in
// starkv_serve/kernels/ keep the reference signatures and call these operators.
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <optional>
#include <vector>

#include "../../include/starkv_hip.h"

namespace {

int dtype_code(const at::Tensor& t) {
    switch (t.scalar_type()) {
        case at::kFloat: return STARKV_F32;
        case at::kHalf: return STARKV_F16;
        case at::kBFloat16: return STARKV_BF16;
        default: TORCH_CHECK(false, "starkv: unsupported dtype ", t.scalar_type());
    }
    return -1;
}

void* stream_of(const at::Tensor& t) { return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check(int rc, const char* what) { TORCH_CHECK(rc == STARKV_OK, "starkv.", what, ": ", starkv_last_error()); }

const int32_t* i32(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.scalar_type() == at::kInt && t.is_contiguous(), "starkv: ", name, " must be contiguous int32");
    return t.data_ptr<int32_t>();
}

int slot_bits(const at::Tensor& s) {
    TORCH_CHECK(s.is_contiguous(), "starkv: slot_mapping must be contiguous");
    if (s.scalar_type() == at::kLong) return 64;
    TORCH_CHECK(s.scalar_type() == at::kInt, "starkv: slot_mapping must be int32 or int64");
    return 32;
}

at::Tensor workspace(const at::Tensor& like, size_t bytes) {
    return at::empty({(int64_t)bytes}, like.options().dtype(at::kByte));
}

// A deferred write's operands and workspace, held from write_kv(deferred) until the
// library has launched the write (the next decode op of this thread, or flush_write):
// the caching allocator may hand out the workspace again only after that launch.
static thread_local std::vector<at::Tensor> t_deferred_hold;

static void release_deferred() { t_deferred_hold.clear(); }

// One bf16/fp16 decode call (paged_decode.py:150-226), at most 1024 requests. A deferred
// write of this thread on the same stream is launched inside it (its operands are then
// released).
void lowrank_decode(const at::Tensor& query, const at::Tensor& kv_cache, const at::Tensor& block_table,
                    const at::Tensor& seq_lens, int64_t max_seq_len, const at::Tensor& k_up, const at::Tensor& k_ranks,
                    const at::Tensor& k_head_offsets, int64_t k_width, int64_t v_col, const at::Tensor& v_up_by_q,
                    const at::Tensor& cos_sin, double scale, const at::Tensor& out) {
    const c10::DeviceGuard guard(query.device());
    const int n = (int)query.size(0), H = (int)query.size(1), Hkv = (int)k_ranks.numel();
    const int v_rank = (int)v_up_by_q.size(1), kind = dtype_code(kv_cache);
    const int grid = starkv_decode_grid_for(kind, n, H, Hkv, (int)k_width, v_rank, (int)max_seq_len);
    TORCH_CHECK(grid > 0, "starkv.lowrank_decode: no grid for ", n, " requests");
    const at::Tensor ws = workspace(
        query, starkv_decode_workspace_bytes(kind, n, H, Hkv, (int)k_width, v_rank, (int)max_seq_len, grid));
    const int rc = starkv_lowrank_decode(stream_of(query), query.data_ptr(), query.stride(0), query.stride(1),
                                dtype_code(query), kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), kind,
                                (int)kv_cache.size(1), i32(block_table, "block_table"), block_table.stride(0),
                                block_table.stride(1), i32(seq_lens, "seq_lens"), n, H, Hkv, (int)max_seq_len,
                                k_up.data_ptr(), k_up.stride(0), dtype_code(k_up), i32(k_ranks, "k_ranks"),
                                i32(k_head_offsets, "k_head_offsets"), (int)k_width, (int)v_col,
                                v_up_by_q.data_ptr(), v_up_by_q.stride(0), v_up_by_q.stride(1), dtype_code(v_up_by_q),
                                v_rank, cos_sin.data_ptr(), cos_sin.stride(0), dtype_code(cos_sin), (float)scale,
                                out.data_ptr(), out.stride(0), out.stride(1), dtype_code(out), ws.data_ptr(),
                                (size_t)ws.numel(), grid);
    release_deferred();
    check(rc, "lowrank_decode");
}

// One 3.2-bit decode call (paged_quant.py:357-411), at most 1024 requests; a deferred
// write as in lowrank_decode.
void quant_decode(const at::Tensor& query, const at::Tensor& kv_cache, const at::Tensor& block_table,
                  const at::Tensor& seq_lens, int64_t max_seq_len, int64_t k_width, int64_t v_rank, int64_t row_bytes,
                  const at::Tensor& k_up, const at::Tensor& tile_head, const at::Tensor& tile_nout,
                  const at::Tensor& tile_last, const at::Tensor& v_up_by_q, const at::Tensor& cos_sin, double scale,
                  const at::Tensor& out, int64_t row_k_width, int64_t row_num_heads, int64_t head0, int64_t k_lane0) {
    const c10::DeviceGuard guard(query.device());
    TORCH_CHECK(kv_cache.scalar_type() == at::kByte, "starkv.quant_decode: the cache is uint8 rows");
    const int n = (int)query.size(0), H = (int)query.size(1);
    const int grid = starkv_decode_grid_for(STARKV_CACHE_Q3_2, n, H, H, (int)k_width, (int)v_rank, (int)max_seq_len);
    TORCH_CHECK(grid > 0, "starkv.quant_decode: no grid for ", n, " requests");
    const size_t need = starkv_quant_group_workspace_bytes(n, (int)row_k_width, (int)row_num_heads, (int)v_rank,
                                                           (int)head0, H, (int)k_lane0, (int)k_width,
                                                           (int)max_seq_len, grid);
    TORCH_CHECK(need > 0, "starkv.quant_decode: heads [", head0, ", ", head0 + H, ") with K lanes [", k_lane0, ", ",
                k_lane0 + k_width, ") do not fit a layer of ", row_num_heads, " heads and K width ", row_k_width);
    const at::Tensor ws = workspace(query, need);
    const int rc = starkv_quant_decode_group(
              stream_of(query), query.data_ptr(), query.stride(0), query.stride(1), dtype_code(query),
              kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0), kv_cache.stride(1), (int)kv_cache.size(1),
              i32(block_table, "block_table"), block_table.stride(0), block_table.stride(1), i32(seq_lens, "seq_lens"),
              n, H, (int)max_seq_len, (int)k_width, (int)v_rank, (int)row_bytes, k_up.data_ptr(), k_up.stride(0),
              dtype_code(k_up), i32(tile_head, "tile_head"), i32(tile_nout, "tile_nout"), i32(tile_last, "tile_last"),
              v_up_by_q.data_ptr(), v_up_by_q.stride(0), v_up_by_q.stride(1), dtype_code(v_up_by_q),
              cos_sin.data_ptr(), cos_sin.stride(0), dtype_code(cos_sin), (float)scale, out.data_ptr(), out.stride(0),
              out.stride(1), dtype_code(out), ws.data_ptr(), (size_t)ws.numel(), grid, (int)row_k_width,
              (int)row_num_heads, (int)head0, (int)k_lane0);
    release_deferred();
    check(rc, "quant_decode");
}

// 3.2-bit quantize + scatter (paged_quant.py:205-216).
void pack_kv(const at::Tensor& k_codes, const at::Tensor& v_codes, const at::Tensor& cache,
             const at::Tensor& slot_mapping, int64_t num_kv_heads, const at::Tensor& k_ranks,
             const at::Tensor& k_offsets, const at::Tensor& k_nouts, int64_t k_width, int64_t v_rank,
             int64_t row_bytes) {
    const c10::DeviceGuard guard(cache.device());
    TORCH_CHECK(cache.scalar_type() == at::kByte, "starkv.pack_kv: the cache is uint8 rows");
    check(starkv_pack_kv(stream_of(cache), k_codes.data_ptr(), k_codes.stride(0), v_codes.data_ptr(),
                         v_codes.stride(0), dtype_code(k_codes), cache.data_ptr<uint8_t>(), cache.stride(0),
                         cache.stride(1), (int)cache.size(1), cache.size(0), slot_mapping.data_ptr(),
                         slot_bits(slot_mapping), (int)k_codes.size(0), (int)num_kv_heads, i32(k_ranks, "k_ranks"),
                         i32(k_offsets, "k_offsets"), i32(k_nouts, "k_nouts"), (int)k_width, (int)v_rank,
                         (int)row_bytes),
          "pack_kv");
}

// bf16/fp16 codes scatter (attention.py:179-184).
void write_codes(const at::Tensor& key, const at::Tensor& value, const at::Tensor& kv_cache,
                 const at::Tensor& slot_mapping) {
    const c10::DeviceGuard guard(kv_cache.device());
    check(starkv_write_codes(stream_of(kv_cache), key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                             dtype_code(key), kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1),
                             dtype_code(kv_cache), (int)kv_cache.size(1), kv_cache.size(0), slot_mapping.data_ptr(),
                             slot_bits(slot_mapping), (int)key.size(0), (int)key.size(1), (int)value.size(1)),
          "write_codes");
}

// The codes' GEMM fused with the cache write (model.py:71 + attention.py:179-188). With
// row_bytes > 0 the cache holds 3.2-bit rows of num_kv_heads heads (k_ranks, k_offsets,
// k_nouts as pack_kv); codes, when given, receives the rounded codes.
void write_kv(const at::Tensor& hidden, const at::Tensor& kv_down, int64_t k_width, const at::Tensor& kv_cache,
              const at::Tensor& slot_mapping, int64_t num_kv_heads, const std::optional<at::Tensor>& k_ranks,
              const std::optional<at::Tensor>& k_offsets, const std::optional<at::Tensor>& k_nouts, int64_t row_bytes,
              const std::optional<at::Tensor>& codes, bool deferred) {
    const c10::DeviceGuard guard(hidden.device());
    const int n = (int)hidden.size(0), hs = (int)hidden.size(1), width = (int)kv_down.size(0);
    const bool q = row_bytes > 0;
    TORCH_CHECK(!q || (k_ranks && k_offsets && k_nouts), "starkv.write_kv: 3.2-bit rows need the K head tables");
    const at::Tensor ws = workspace(hidden, starkv_write_kv_workspace_bytes(n, width, hs));
    // Either call launches a write still pending from before, whose operands are then free.
    std::vector<at::Tensor> held;
    held.swap(t_deferred_hold);
    auto* fn = deferred ? &starkv_write_kv_deferred : &starkv_write_kv;
    check(fn(stream_of(hidden), hidden.data_ptr(), hidden.stride(0), kv_down.data_ptr(),
                          kv_down.stride(0), dtype_code(hidden), n, hs, (int)k_width, width - (int)k_width,
                          kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), q ? 0 : dtype_code(kv_cache),
                          (int)kv_cache.size(1), kv_cache.size(0), slot_mapping.data_ptr(), slot_bits(slot_mapping),
                          q ? (int)num_kv_heads : 0, q ? i32(*k_ranks, "k_ranks") : nullptr,
                          q ? i32(*k_offsets, "k_offsets") : nullptr, q ? i32(*k_nouts, "k_nouts") : nullptr,
                          q ? (int)row_bytes : 0, codes ? codes->data_ptr() : nullptr, codes ? codes->stride(0) : 0,
                          ws.data_ptr(), (size_t)ws.numel()),
          "write_kv");
    if (deferred && n > 0) {
        t_deferred_hold = {hidden, kv_down, slot_mapping, ws};
        for (const auto* t : {&k_ranks, &k_offsets, &k_nouts, &codes})
            if (*t) t_deferred_hold.push_back(**t);
    }
}

// Launches this thread's deferred write, if any.
void flush_write() {
    const int rc = starkv_flush_write();
    release_deferred();
    check(rc, "flush_write");
}

// q folded into U (paged_quant.py:241-255): ab [n, k_width, 128] fp16.
void fold_q(const at::Tensor& q, const at::Tensor& k_up, const at::Tensor& head_of_lane, double scale,
            const at::Tensor& ab) {
    const c10::DeviceGuard guard(q.device());
    TORCH_CHECK(ab.scalar_type() == at::kHalf && ab.is_contiguous(), "starkv.fold_q: ab must be contiguous fp16");
    check(starkv_fold_q(stream_of(q), q.data_ptr(), q.stride(0), q.stride(1), dtype_code(q), k_up.data_ptr(),
                        k_up.stride(0), dtype_code(k_up), i32(head_of_lane, "head_of_lane"), (int)q.size(0),
                        (int)k_up.size(0), (float)scale, ab.data_ptr()),
          "fold_q");
}

// Uncompressed paged decode (the stock attention of uncompressed layers).
void stock_decode(const at::Tensor& query, const at::Tensor& k_cache, const at::Tensor& v_cache,
                  const at::Tensor& block_table, const at::Tensor& seq_lens, int64_t max_seq_len, double scale,
                  const at::Tensor& out) {
    const c10::DeviceGuard guard(query.device());
    const int n = (int)query.size(0), H = (int)query.size(1), Hkv = (int)k_cache.size(2);
    TORCH_CHECK(k_cache.strides() == v_cache.strides(), "starkv.stock_decode: K and V caches must share strides");
    const at::Tensor ws = workspace(query, starkv_stock_decode_workspace_bytes(n, H, Hkv, (int)max_seq_len));
    check(starkv_stock_decode(stream_of(query), query.data_ptr(), query.stride(0), query.stride(1), dtype_code(query),
                              k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
                              k_cache.stride(2), dtype_code(k_cache), (int)k_cache.size(1),
                              i32(block_table, "block_table"), block_table.stride(0), block_table.stride(1),
                              i32(seq_lens, "seq_lens"), n, H, Hkv, (int)max_seq_len, (float)scale, out.data_ptr(),
                              out.stride(0), out.stride(1), dtype_code(out), ws.data_ptr(), (size_t)ws.numel()),
          "stock_decode");
}

// Uncompressed K/V scatter (vLLM's reshape_and_cache).
void stock_write(const at::Tensor& key, const at::Tensor& value, const at::Tensor& k_cache, const at::Tensor& v_cache,
                 const at::Tensor& slot_mapping) {
    const c10::DeviceGuard guard(key.device());
    TORCH_CHECK(k_cache.strides() == v_cache.strides(), "starkv.stock_write: K and V caches must share strides");
    check(starkv_stock_write(stream_of(key), key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(),
                             value.stride(0), value.stride(1), dtype_code(key), k_cache.data_ptr(), v_cache.data_ptr(),
                             k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), (int)k_cache.size(1),
                             k_cache.size(0), slot_mapping.data_ptr(), slot_bits(slot_mapping), (int)key.size(0),
                             (int)key.size(1)),
          "stock_write");
}

// Dense causal prefill attention over lifted K / V (attention.py:219-251's attention).
void prefill(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value, const at::Tensor& cu_seqlens,
             const at::Tensor& blocks, double scale, const at::Tensor& out) {
    const c10::DeviceGuard guard(query.device());
    TORCH_CHECK(key.strides() == value.strides(), "starkv.prefill: K and V must share strides");
    TORCH_CHECK(blocks.dim() == 2 && blocks.size(1) == 2, "starkv.prefill: blocks must be [num_blocks, 2]");
    check(starkv_prefill_attention(stream_of(query), query.data_ptr(), query.stride(0), query.stride(1),
                                   dtype_code(query), key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1),
                                   dtype_code(key), i32(cu_seqlens, "cu_seqlens"), i32(blocks, "blocks"),
                                   (int)blocks.size(0), (int)query.size(1), (int)key.size(1), (int)query.size(2),
                                   (float)scale, out.data_ptr(), out.stride(0), out.stride(1), dtype_code(out)),
          "prefill");
}

}  // namespace

TORCH_LIBRARY(starkv, m) {
    m.def("lowrank_decode(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, int max_seq_len, "
          "Tensor k_up, Tensor k_ranks, Tensor k_head_offsets, int k_width, int v_col, Tensor v_up_by_q, "
          "Tensor cos_sin, float scale, Tensor(a!) out) -> ()");
    m.def("quant_decode(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, int max_seq_len, "
          "int k_width, int v_rank, int row_bytes, Tensor k_up, Tensor tile_head, Tensor tile_nout, "
          "Tensor tile_last, Tensor v_up_by_q, Tensor cos_sin, float scale, Tensor(a!) out, int row_k_width, "
          "int row_num_heads, int head0, int k_lane0) -> ()");
    m.def("pack_kv(Tensor k_codes, Tensor v_codes, Tensor(a!) cache, Tensor slot_mapping, int num_kv_heads, "
          "Tensor k_ranks, Tensor k_offsets, Tensor k_nouts, int k_width, int v_rank, int row_bytes) -> ()");
    m.def("write_codes(Tensor key, Tensor value, Tensor(a!) kv_cache, Tensor slot_mapping) -> ()");
    m.def("write_kv(Tensor hidden, Tensor kv_down, int k_width, Tensor(a!) kv_cache, Tensor slot_mapping, "
          "int num_kv_heads, Tensor? k_ranks, Tensor? k_offsets, Tensor? k_nouts, int row_bytes, "
          "Tensor(b!)? codes, bool deferred=False) -> ()");
    m.def("flush_write() -> ()", &flush_write);
    m.def("fold_q(Tensor q, Tensor k_up, Tensor head_of_lane, float scale, Tensor(a!) ab) -> ()");
    m.def("stock_decode(Tensor query, Tensor k_cache, Tensor v_cache, Tensor block_table, Tensor seq_lens, "
          "int max_seq_len, float scale, Tensor(a!) out) -> ()");
    m.def("stock_write(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping) -> ()");
    m.def("prefill(Tensor query, Tensor key, Tensor value, Tensor cu_seqlens, Tensor blocks, float scale, "
          "Tensor(a!) out) -> ()");
}

TORCH_LIBRARY_IMPL(starkv, CUDA, m) {
    m.impl("lowrank_decode", &lowrank_decode);
    m.impl("quant_decode", &quant_decode);
    m.impl("pack_kv", &pack_kv);
    m.impl("write_codes", &write_codes);
    m.impl("write_kv", &write_kv);
    m.impl("fold_q", &fold_q);
    m.impl("stock_decode", &stock_decode);
    m.impl("stock_write", &stock_write);
    m.impl("prefill", &prefill);
}
