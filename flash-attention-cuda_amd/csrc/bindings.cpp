// flashattn_cuda._C — the pybind11 surface of the reference
// (csrc/bindings.cpp:10-134 of shrvan30/flash-attention-cuda) on top of the
// C ABI in include/flashattn_hip.h.
//
// Kept identical to the reference: function names, keyword names, argument
// meaning, TORCH_CHECK validation order and message text (the tests match on
// "must be fp16", "must be a CUDA tensor", "must be 4-D", "must be
// contiguous", "head_dim", "identical shapes", "exactly one query row",
// "seq_lens must be int32", "seq_lens must be 1-D"), output allocation with
// empty_like(q), asynchronous launch on the current stream, no host sync.
// Added: head_dim 128 for prefill / decode / append_kv (the head size is
// read from the tensors; `head_dim` stays 64, `head_dims` lists both), a
// device guard for inputs that live on a non-current device, the
// fp32-output parity hooks `_prefill_fp32` / `_decode_fp32`, and grouped-query
// variants `prefill_gqa` / `decode_gqa` (K/V with fewer heads than Q). The v1
// legacy_naive / legacy_tiled / legacy_fused kernels (csrc/legacy/) keep
// their own checks and messages (legacy_ops.cu:19-35).
//
// Torch-ROCm calls the HIP device "cuda", so `is_cuda()` is the right check
// and the reference's messages stay verbatim; the device guard and stream
// lookup use torch's "masquerading as CUDA" HIP classes for the same reason.

#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <string>
#include <vector>

#include "flashattn_hip.h"

namespace {

constexpr int kHeadDim = FA_HEAD_DIM;

// flash_common.h:43-62 of the reference. The head size may also be 128 here
// (the reference's named next step, README.md:397); any other size fails
// with a "head_dim" message as in the reference.
void check_bhnd(const at::Tensor &t, const char *name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.scalar_type() == at::kHalf, name, " must be fp16 (got ",
              t.scalar_type(), ")");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous row-major");
  TORCH_CHECK(t.dim() == 4, name, " must be 4-D (B, H, N, ", kHeadDim,
              "), got ", t.dim(), "-D");
  TORCH_CHECK(t.size(3) == kHeadDim || t.size(3) == 128, name,
              " must have head_dim == ", kHeadDim, " (or 128), got ", t.size(3));
}

void check_status(int rc) {
  TORCH_CHECK(rc == FA_OK, "flashattn_hip: ", fa_last_error());
}

void *stream_of(const at::Tensor &t) {
  return static_cast<void *>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

// bindings.cpp:10-27. With `grouped`, k and v are [B, H_kv, S, 64] with
// H_kv dividing H (grouped-query attention, no reference counterpart);
// otherwise all three shapes must be identical, as in the reference.
at::Tensor prefill_impl(const at::Tensor &q, const at::Tensor &k,
                        const at::Tensor &v, bool causal, double scale,
                        bool out_f32, bool grouped = false) {
  check_bhnd(q, "q");
  check_bhnd(k, "k");
  check_bhnd(v, "v");
  if (grouped) {
    TORCH_CHECK(k.sizes() == v.sizes(),
                "prefill_gqa expects k and v to have identical shapes, got k=", k.sizes(),
                " v=", v.sizes());
    TORCH_CHECK(q.size(0) == k.size(0) && q.size(2) == k.size(2),
                "prefill_gqa expects q and k/v to agree on batch and sequence length, got q=",
                q.sizes(), " k=", k.sizes());
    TORCH_CHECK(k.size(1) > 0 && q.size(1) % k.size(1) == 0,
                "prefill_gqa expects the K/V head count to divide the query head count, "
                "got H=", q.size(1), " H_kv=", k.size(1));
    TORCH_CHECK(q.size(3) == k.size(3),
                "prefill_gqa expects q and k/v to have the same head_dim, got ", q.size(3),
                " and ", k.size(3));
  } else {
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(),
                "prefill expects q, k and v to have identical shapes, got q=",
                q.sizes(), " k=", k.sizes(), " v=", v.sizes());
  }
  TORCH_CHECK(q.device() == k.device() && q.device() == v.device(),
              "q, k and v must live on the same device");
  TORCH_CHECK(q.size(2) > 0, "sequence length must be > 0");
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");

  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor o = out_f32 ? at::empty(q.sizes(), q.options().dtype(at::kFloat))
                         : at::empty_like(q);
  if (q.numel() == 0) return o;
  const size_t ws_bytes = fa_prefill_workspace_bytes(
      static_cast<int>(q.size(0)), static_cast<int>(q.size(1)),
      static_cast<int>(q.size(2)), causal ? 1 : 0);
  at::Tensor ws;
  if (ws_bytes > 0)
    ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  check_status(fa_prefill_hd(q.const_data_ptr(), k.const_data_ptr(),
                             v.const_data_ptr(), o.data_ptr(),
                             out_f32 ? FA_OUT_F32 : FA_OUT_F16,
                             static_cast<int>(q.size(0)),
                             static_cast<int>(q.size(1)),
                             static_cast<int>(k.size(1)),
                             static_cast<int>(q.size(2)), static_cast<int>(q.size(3)),
                             causal ? 1 : 0, static_cast<float>(scale),
                             ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                             stream_of(q)));
  return o;
}

at::Tensor prefill(const at::Tensor &q, const at::Tensor &k,
                   const at::Tensor &v, bool causal, double scale) {
  return prefill_impl(q, k, v, causal, scale, false);
}

at::Tensor prefill_fp32(const at::Tensor &q, const at::Tensor &k,
                        const at::Tensor &v, bool causal, double scale) {
  return prefill_impl(q, k, v, causal, scale, true);
}

at::Tensor prefill_gqa(const at::Tensor &q, const at::Tensor &k,
                       const at::Tensor &v, bool causal, double scale) {
  return prefill_impl(q, k, v, causal, scale, false, true);
}

at::Tensor prefill_gqa_fp32(const at::Tensor &q, const at::Tensor &k,
                            const at::Tensor &v, bool causal, double scale) {
  return prefill_impl(q, k, v, causal, scale, true, true);
}

// bindings.cpp:36-70. With `grouped`, the caches are [B, H_kv, Lmax, 64]
// with H_kv dividing H (no reference counterpart).
at::Tensor decode_core(const at::Tensor &q, const at::Tensor &k_cache,
                       const at::Tensor &v_cache, const at::Tensor &seq_lens,
                       double scale, int64_t split_size, bool out_f32,
                       bool grouped = false) {
  check_bhnd(q, "q");
  check_bhnd(k_cache, "k_cache");
  check_bhnd(v_cache, "v_cache");

  TORCH_CHECK(q.size(2) == 1, "decode expects exactly one query row, got ",
              q.size(2));
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(),
              "k_cache and v_cache must have identical shapes, got ",
              k_cache.sizes(), " and ", v_cache.sizes());
  if (grouped) {
    TORCH_CHECK(q.size(0) == k_cache.size(0) && k_cache.size(1) > 0 &&
                    q.size(1) % k_cache.size(1) == 0,
                "decode_gqa expects q and the caches to agree on batch and the K/V head "
                "count to divide the query head count, got q=",
                q.sizes(), " cache=", k_cache.sizes());
  } else {
    TORCH_CHECK(q.size(0) == k_cache.size(0) && q.size(1) == k_cache.size(1),
                "q and the caches must agree on batch and head count, got q=",
                q.sizes(), " cache=", k_cache.sizes());
  }
  TORCH_CHECK(q.size(3) == k_cache.size(3),
              "q and the caches must have the same head_dim, got ", q.size(3), " and ",
              k_cache.size(3));
  TORCH_CHECK(k_cache.size(2) > 0, "cache length must be > 0");

  TORCH_CHECK(seq_lens.is_cuda(), "seq_lens", " must be a CUDA tensor");
  TORCH_CHECK(seq_lens.is_contiguous(), "seq_lens",
              " must be contiguous row-major");
  TORCH_CHECK(seq_lens.scalar_type() == at::kInt,
              "seq_lens must be int32 (got ", seq_lens.scalar_type(), ")");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.size(0) == q.size(0),
              "seq_lens must be 1-D of length B=", q.size(0), ", got ",
              seq_lens.sizes());
  TORCH_CHECK(q.device() == k_cache.device() &&
                  q.device() == v_cache.device() &&
                  q.device() == seq_lens.device(),
              "q, caches and seq_lens must live on the same device");
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  TORCH_CHECK(split_size >= 0 && split_size <= (int64_t{1} << 30),
              "decode split size must be >= 0, got ", split_size);

  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor o = out_f32 ? at::empty(q.sizes(), q.options().dtype(at::kFloat))
                         : at::empty_like(q);
  if (q.numel() == 0) return o;
  const int batch = static_cast<int>(q.size(0));
  const int heads = static_cast<int>(q.size(1));
  const int kv_heads = static_cast<int>(k_cache.size(1));
  const int max_seq = static_cast<int>(k_cache.size(2));
  const int split = static_cast<int>(split_size);
  const int head_dim = static_cast<int>(q.size(3));
  const size_t ws_bytes =
      fa_decode_hd_workspace_bytes(batch, heads, kv_heads, max_seq, head_dim, split);
  // 0 bytes: the whole-sequence kernel needs no workspace, unless the query
  // failed (then fa_last_error() says why).
  check_status(ws_bytes > 0 || fa_last_error()[0] == '\0' ? FA_OK : FA_ERR_INVALID_ARGUMENT);
  // Transient, stream-ordered workspace from the caching allocator
  // (decode.cu:215-219 of the reference), only when the split-K partials need it.
  at::Tensor ws;
  if (ws_bytes > 0)
    ws = at::empty({static_cast<int64_t>(ws_bytes / sizeof(float))},
                   q.options().dtype(at::kFloat));
  check_status(fa_decode_hd(q.const_data_ptr(), k_cache.const_data_ptr(),
                            v_cache.const_data_ptr(),
                            seq_lens.const_data_ptr<int32_t>(), o.data_ptr(),
                            out_f32 ? FA_OUT_F32 : FA_OUT_F16, batch, heads, kv_heads,
                            max_seq, head_dim, static_cast<float>(scale), split,
                            ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
  return o;
}

at::Tensor decode_impl(const at::Tensor &q, const at::Tensor &k_cache,
                       const at::Tensor &v_cache, const at::Tensor &seq_lens,
                       double scale, int64_t split_size) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, split_size, false);
}

// bindings.cpp:72-76.
at::Tensor decode(const at::Tensor &q, const at::Tensor &k_cache,
                  const at::Tensor &v_cache, const at::Tensor &seq_lens,
                  double scale) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, 0, false);
}

at::Tensor decode_fp32(const at::Tensor &q, const at::Tensor &k_cache,
                       const at::Tensor &v_cache, const at::Tensor &seq_lens,
                       double scale, int64_t split_size) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, split_size, true);
}

at::Tensor decode_gqa(const at::Tensor &q, const at::Tensor &k_cache,
                      const at::Tensor &v_cache, const at::Tensor &seq_lens,
                      double scale) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, 0, false, true);
}

at::Tensor decode_gqa_fp32(const at::Tensor &q, const at::Tensor &k_cache,
                           const at::Tensor &v_cache, const at::Tensor &seq_lens,
                           double scale, int64_t split_size) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, split_size, true, true);
}

at::Tensor decode_gqa_with_split(const at::Tensor &q, const at::Tensor &k_cache,
                                 const at::Tensor &v_cache, const at::Tensor &seq_lens,
                                 double scale, int64_t split_size) {
  return decode_core(q, k_cache, v_cache, seq_lens, scale, split_size, false, true);
}

// KV-cache append (no reference counterpart: its caller's cache write).
// k_cache, v_cache [B, H_kv, Lmax, 64], k, v [B, H_kv, 1, 64], seq_lens [B]
// int32, all on one device; updates the caches and seq_lens in place.
void append_kv(const at::Tensor &k_cache, const at::Tensor &v_cache, const at::Tensor &k,
               const at::Tensor &v, const at::Tensor &seq_lens) {
  check_bhnd(k_cache, "k_cache");
  check_bhnd(v_cache, "v_cache");
  check_bhnd(k, "k");
  check_bhnd(v, "v");
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(),
              "k_cache and v_cache must have identical shapes, got ", k_cache.sizes(), " and ",
              v_cache.sizes());
  TORCH_CHECK(k.size(2) == 1 && k.sizes() == v.sizes() && k.size(0) == k_cache.size(0) &&
                  k.size(1) == k_cache.size(1) && k.size(3) == k_cache.size(3),
              "append_kv expects k and v of shape [B, H_kv, 1, head_dim] matching the caches, "
              "got k=", k.sizes(), " v=", v.sizes(), " cache=", k_cache.sizes());
  TORCH_CHECK(k_cache.size(2) > 0, "cache length must be > 0");
  TORCH_CHECK(seq_lens.is_cuda(), "seq_lens", " must be a CUDA tensor");
  TORCH_CHECK(seq_lens.is_contiguous(), "seq_lens", " must be contiguous row-major");
  TORCH_CHECK(seq_lens.scalar_type() == at::kInt,
              "seq_lens must be int32 (got ", seq_lens.scalar_type(), ")");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.size(0) == k_cache.size(0),
              "seq_lens must be 1-D of length B=", k_cache.size(0), ", got ", seq_lens.sizes());
  TORCH_CHECK(k_cache.device() == v_cache.device() && k_cache.device() == k.device() &&
                  k_cache.device() == v.device() && k_cache.device() == seq_lens.device(),
              "caches, k, v and seq_lens must live on the same device");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(k_cache.device());
  if (k_cache.numel() == 0) return;
  check_status(fa_kv_append_hd(k_cache.data_ptr(), v_cache.data_ptr(), k.const_data_ptr(),
                               v.const_data_ptr(), seq_lens.data_ptr<int32_t>(),
                               static_cast<int>(k_cache.size(0)),
                               static_cast<int>(k_cache.size(1)),
                               static_cast<int>(k_cache.size(2)),
                               static_cast<int>(k_cache.size(3)), stream_of(k_cache)));
}

// bindings.cpp:80-97.
py::list occupancy_report() {
  // The first call counts the rows, the second fills them.
  int n = 0;
  check_status(fa_occupancy_report(nullptr, 0, &n));
  std::vector<fa_occupancy_entry> rows(static_cast<size_t>(n));
  check_status(fa_occupancy_report(rows.data(), n, &n));
  py::list out;
  for (int i = 0; i < n && i < static_cast<int>(rows.size()); ++i) {
    py::dict row;
    row["kernel"] = std::string(rows[i].kernel);
    row["threads_per_block"] = rows[i].threads_per_block;
    row["registers_per_thread"] = rows[i].registers_per_thread;
    row["shared_bytes_per_block"] = rows[i].shared_bytes_per_block;
    row["max_active_blocks_per_sm"] = rows[i].max_active_blocks_per_sm;
    row["theoretical_occupancy"] = rows[i].theoretical_occupancy;
    out.append(row);
  }
  return out;
}

// csrc/legacy/legacy_ops.cu:19-51: the v1 single-head fp32 kernels, with the
// reference's check order and messages; the output is empty_like(q).
void check_legacy_inputs(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(),
              "legacy kernels expect CUDA tensors");
  TORCH_CHECK(q.scalar_type() == at::kFloat && k.scalar_type() == at::kFloat &&
                  v.scalar_type() == at::kFloat,
              "legacy kernels are fp32 only");
  TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(),
              "legacy kernels expect contiguous tensors");
  TORCH_CHECK(q.dim() == 2 && k.dim() == 2 && v.dim() == 2,
              "legacy kernels are single-head: expected (N, ", kHeadDim, ") tensors");
  TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(),
              "legacy kernels expect identical q/k/v shapes");
  TORCH_CHECK(q.size(1) == kHeadDim, "legacy kernels expect head_dim == ", kHeadDim);
  TORCH_CHECK(q.device() == k.device() && q.device() == v.device(),
              "legacy kernels expect q, k and v on the same device");
}

at::Tensor legacy_impl(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                       int variant) {
  check_legacy_inputs(q, k, v);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor o = at::empty_like(q);
  if (q.size(0) == 0) return o;  // empty tensors carry no data pointer
  TORCH_CHECK(q.size(0) < (int64_t{1} << 31) / kHeadDim, "legacy kernels: too many rows");
  check_status(fa_legacy_attention(q.const_data_ptr<float>(), k.const_data_ptr<float>(),
                                   v.const_data_ptr<float>(), o.data_ptr<float>(),
                                   static_cast<int>(q.size(0)), variant, stream_of(q)));
  return o;
}

at::Tensor legacy_naive(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v) {
  return legacy_impl(q, k, v, FA_LEGACY_NAIVE);
}
at::Tensor legacy_tiled(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v) {
  return legacy_impl(q, k, v, FA_LEGACY_TILED);
}
at::Tensor legacy_fused(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v) {
  return legacy_impl(q, k, v, FA_LEGACY_FUSED);
}

int choose_decode_split(int max_seq, int batch, int heads, int min_blocks) {
  return fa_choose_decode_split(max_seq, batch, heads, min_blocks);
}

}  // namespace

// bindings.cpp:110-134.
PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Batched multi-head causal FlashAttention kernels for head_dim=64 "
            "(MI355X / gfx950)";
  m.attr("head_dim") = kHeadDim;
  // Head sizes the kernels accept (128: no reference counterpart).
  m.attr("head_dims") = py::make_tuple(kHeadDim, 128);

  m.def("prefill", &prefill,
        "Full-sequence attention (fp16 in/out, fp32 accum)", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("causal"), py::arg("scale"));
  m.def("decode", &decode, "Single-query attention against a KV cache",
        py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("seq_lens"), py::arg("scale"));
  m.def("occupancy_report", &occupancy_report,
        "Theoretical occupancy of each kernel at its launch configuration");
  m.def("choose_decode_split", &choose_decode_split,
        "Chunk size decode would pick for this shape and block target",
        py::arg("max_seq"), py::arg("batch"), py::arg("heads"),
        py::arg("min_blocks"));
  // Benchmark hook: forces the split-K chunk size instead of choosing it.
  m.def("_decode_with_split", &decode_impl, py::arg("q"), py::arg("k_cache"),
        py::arg("v_cache"), py::arg("seq_lens"), py::arg("scale"),
        py::arg("split_size"));
  // Parity hooks: the same kernels with an fp32 epilogue (no final rounding).
  m.def("_prefill_fp32", &prefill_fp32, py::arg("q"), py::arg("k"),
        py::arg("v"), py::arg("causal"), py::arg("scale"));
  m.def("_decode_fp32", &decode_fp32, py::arg("q"), py::arg("k_cache"),
        py::arg("v_cache"), py::arg("seq_lens"), py::arg("scale"),
        py::arg("split_size") = 0);

  // Grouped-query attention (no reference counterpart): k/v (or the caches)
  // carry H_kv heads, H_kv dividing H; query head h reads K/V head
  // h / (H / H_kv), the same pairing as repeat_interleave(k, H / H_kv, dim=1).
  m.def("prefill_gqa", &prefill_gqa,
        "Full-sequence attention with H_kv <= H K/V heads (fp16 in/out, fp32 accum)",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal"), py::arg("scale"));
  m.def("decode_gqa", &decode_gqa,
        "Single-query attention against a KV cache with H_kv <= H K/V heads",
        py::arg("q"), py::arg("k_cache"), py::arg("v_cache"), py::arg("seq_lens"),
        py::arg("scale"));
  m.def("_decode_gqa_with_split", &decode_gqa_with_split, py::arg("q"),
        py::arg("k_cache"), py::arg("v_cache"), py::arg("seq_lens"), py::arg("scale"),
        py::arg("split_size"));
  m.def("_prefill_gqa_fp32", &prefill_gqa_fp32, py::arg("q"), py::arg("k"),
        py::arg("v"), py::arg("causal"), py::arg("scale"));
  // KV-cache append (no reference counterpart): writes k, v at row
  // seq_lens[b] of the caches and advances seq_lens, on the device.
  m.def("append_kv", &append_kv,
        "Write one token's K/V at row seq_lens[b] of the caches and advance seq_lens",
        py::arg("k_cache"), py::arg("v_cache"), py::arg("k"), py::arg("v"),
        py::arg("seq_lens"));
  m.def("_decode_gqa_fp32", &decode_gqa_fp32, py::arg("q"), py::arg("k_cache"),
        py::arg("v_cache"), py::arg("seq_lens"), py::arg("scale"),
        py::arg("split_size") = 0);

  // bindings.cpp:131-133: the v1 kernels, (N, 64) fp32, one head, no mask.
  m.def("legacy_naive", &legacy_naive, "v1 naive kernel (N, 64) fp32");
  m.def("legacy_tiled", &legacy_tiled, "v1 tiled kernel (N, 64) fp32");
  m.def("legacy_fused", &legacy_fused, "v1 fused kernel (N, 64) fp32");
}
