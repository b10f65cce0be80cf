// PyTorch-ROCm operator registration of the cqgdn C ABI: TORCH_LIBRARY(cqgdn, m).
//
// The Python host mirror (cqgdn/gated_delta_net.py, cqgdn/events.py) keeps the reference's
// contract checks and error texts (ops/gated_delta_net.py:217-352); the per-step calls then go
// through these ops, which allocate their outputs with the tensors' allocator, enqueue on the
// current HIP stream of the tensors' device (ops/gated_delta_net.py runs its ops on the current
// NPU stream the same way) and turn the library's error codes into Python exceptions:
// CQGDN_EINVAL -> ValueError, CQGDN_EUNSUPPORTED -> NotImplementedError, CQGDN_EHIP -> RuntimeError.
// One op call replaces the Python-level allocations, pointer and stream lookups and the ctypes
// call of each launch; the decode ops also run the reference's contract checks here.  The ops are
// registered for the CUDA dispatch key, which is what PyTorch-ROCm tensors on an AMD GPU carry;
// nothing computes on the CPU (no fallback).
//
// Schemas (T events, H heads, time-first [1,T,H,128] q/k/v of one dtype, bf16 or fp16 (which
// sets CQGDN_FP16; outputs and gradients take that dtype), fp32 [1,T,H] g/beta):
//   fwd(q, k, v, g, beta, table, doc, scale, flags, initial_state?, want_state) -> (o, state, ws)
//       cqgdn_fwd; o is empty with CQGDN_NO_OUTPUT, state empty unless want_state
//   bwd(q, k, v, g, beta, dy, table, doc, scale, flags, ws?) -> (dq, dk, dv, dg, dbeta)
//       cqgdn_bwd with the forward's workspace, or cqgdn_bwd_recompute without one
//   recurrent(q, k, v, g, beta, state!, out!, scale) -> ()
//       cqgdn_recurrent on [N,t,H,128] (or [t,H,128]) q/k/v/out, value-first fp32 state in place
//   layer_decode_step(proj, conv_w, A_log, dt_bias, norm_w, conv_history!, state!, heads, key_heads,
//                     eps, scale) -> out
//       cqgdn_layer_decode_step on [N,2,P] projection rows; history and state in place

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "cqgdn.h"

namespace {

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check(int rc, const char* what) {
  if (rc == CQGDN_OK) return;
  TORCH_CHECK_VALUE(rc != CQGDN_EINVAL, what, ": ", cqgdn_last_error());
  TORCH_CHECK_NOT_IMPLEMENTED(rc != CQGDN_EUNSUPPORTED, what, ": ", cqgdn_last_error());
  TORCH_CHECK(false, what, ": ", cqgdn_last_error());
}

const void* cptr(const at::Tensor& t) { return t.defined() && t.numel() ? t.data_ptr() : nullptr; }
void* mptr(const at::Tensor& t) { return t.defined() && t.numel() ? t.data_ptr() : nullptr; }

at::Tensor bytes(size_t n, const at::Tensor& like) {
  return at::empty({(int64_t)(n ? n : 1)}, like.options().dtype(at::kByte));
}

// CQGDN_FP16 follows the tensors' dtype: q, k, v (and dy) share one, bf16 or fp16
unsigned dtype_flag(const at::Tensor& q, std::initializer_list<const at::Tensor*> same) {
  const auto dt = q.scalar_type();
  TORCH_CHECK_VALUE(dt == at::kBFloat16 || dt == at::kHalf, "QKV must share BF16/FP16 dtype");
  for (const at::Tensor* x : same) TORCH_CHECK_VALUE(x->scalar_type() == dt, "QKV must share BF16/FP16 dtype");
  return dt == at::kHalf ? CQGDN_FP16 : 0u;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                   const at::Tensor& g, const at::Tensor& beta,
                                                   const at::Tensor& table, const at::Tensor& doc, double scale,
                                                   int64_t flags, const std::optional<at::Tensor>& initial_state,
                                                   bool want_state) {
  TORCH_CHECK_VALUE(q.dim() == 4 && q.size(0) == 1 && q.size(3) == CQGDN_HEAD_DIM, "q must be [1,T,H,128]");
  flags = (flags & ~(int64_t)CQGDN_FP16) | dtype_flag(q, {&k, &v});
  const int64_t T = q.size(1), H = q.size(2), n_chunks = table.size(0), n_docs = doc.numel() - 1;
  at::Tensor ws = bytes(cqgdn_fwd_workspace_size(T, (int)H, n_chunks), q);
  at::Tensor o = (flags & CQGDN_NO_OUTPUT) ? at::empty({0}, v.options()) : at::empty_like(v);
  at::Tensor state = want_state ? at::empty({n_docs, H, 128, 128}, q.options().dtype(at::kFloat))
                                : at::empty({0}, q.options().dtype(at::kFloat));
  const at::Tensor init = initial_state.has_value() ? *initial_state : at::Tensor();
  check(cqgdn_fwd(cptr(q), cptr(k), cptr(v), g.data_ptr<float>(), beta.data_ptr<float>(), T, (int)H,
                  table.data_ptr<int32_t>(), n_chunks, doc.data_ptr<int32_t>(), (int)n_docs, (float)scale,
                  (unsigned)flags, init.defined() ? init.data_ptr<float>() : nullptr,
                  want_state ? state.data_ptr<float>() : nullptr, mptr(o), ws.data_ptr(), (size_t)ws.numel(),
                  stream_of(q)),
        "cqgdn_fwd");
  return {o, state, ws};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> bwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& g, const at::Tensor& beta,
    const at::Tensor& dy, const at::Tensor& table, const at::Tensor& doc, double scale, int64_t flags,
    const std::optional<at::Tensor>& fwd_ws) {
  TORCH_CHECK_VALUE(v.dim() == 4 && v.size(0) == 1 && v.size(3) == CQGDN_HEAD_DIM, "v must be [1,T,H,128]");
  flags = (flags & ~(int64_t)CQGDN_FP16) | dtype_flag(q, {&k, &v, &dy});
  const int64_t T = v.size(1), H = v.size(2), n_chunks = table.size(0), n_docs = doc.numel() - 1;
  at::Tensor bws = bytes(cqgdn_bwd_workspace_size(T, (int)H, n_chunks), v);
  at::Tensor dq = at::empty_like(v), dk = at::empty_like(v), dv = at::empty_like(v);
  at::Tensor dg = at::empty_like(g), db = at::empty_like(beta);
  const hipStream_t st = stream_of(v);
  if (fwd_ws.has_value()) {
    const at::Tensor& ws = *fwd_ws;
    check(cqgdn_bwd(cptr(q), cptr(k), cptr(v), g.data_ptr<float>(), beta.data_ptr<float>(), cptr(dy), T, (int)H,
                    table.data_ptr<int32_t>(), n_chunks, doc.data_ptr<int32_t>(), (int)n_docs, (float)scale,
                    (unsigned)flags, ws.data_ptr(), (size_t)ws.numel(), bws.data_ptr(), (size_t)bws.numel(),
                    mptr(dq), mptr(dk), mptr(dv), dg.data_ptr<float>(), db.data_ptr<float>(), st),
          "cqgdn_bwd");
  } else {
    at::Tensor ws = bytes(cqgdn_fwd_workspace_size(T, (int)H, n_chunks), v);
    check(cqgdn_bwd_recompute(cptr(q), cptr(k), cptr(v), g.data_ptr<float>(), beta.data_ptr<float>(), cptr(dy), T,
                              (int)H, table.data_ptr<int32_t>(), n_chunks, doc.data_ptr<int32_t>(), (int)n_docs,
                              (float)scale, (unsigned)flags, ws.data_ptr(), (size_t)ws.numel(), bws.data_ptr(),
                              (size_t)bws.numel(), mptr(dq), mptr(dk), mptr(dv), dg.data_ptr<float>(),
                              db.data_ptr<float>(), st),
          "cqgdn_bwd_recompute");
  }
  return {dq, dk, dv, dg, db};
}

bool on_gpu(const at::Tensor& t) { return t.is_cuda(); }

// ops/gated_delta_net.py:314-352: q, k (l2-normalized), v, out [t,H,128] or [N,t,H,128], one dtype (bf16 or
// fp16, read and written as such); g fp32 (other float types are converted); beta fp32 or bf16; state fp32
// [N,H,V,K] value-first, updated in place.
void recurrent(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& g,
               const at::Tensor& beta, at::Tensor& state, at::Tensor& out, double scale) {
  for (const at::Tensor* x : {&q, &k, &v, &g, &beta, (const at::Tensor*)&state, (const at::Tensor*)&out})
    TORCH_CHECK_VALUE(on_gpu(*x), "the hip GDN backend requires tensors on a ROCm GPU");
  const bool batched = q.dim() == 4;
  TORCH_CHECK_VALUE(batched || q.dim() == 3, "recurrent needs q [t,H,128] or [N,t,H,128]");
  const int64_t n = batched ? q.size(0) : 1, t = q.size(batched ? 1 : 0), h = q.size(batched ? 2 : 1);
  const int64_t d = q.size(q.dim() - 1);
  TORCH_CHECK_VALUE(d == CQGDN_HEAD_DIM && state.sizes() == at::IntArrayRef({n, h, 128, 128}) &&
                        state.scalar_type() == at::kFloat,
                    "recurrent needs d=128 and a value-first fp32 state [N,H,128,128]");
  TORCH_CHECK_VALUE(out.sizes() == q.sizes() && k.sizes() == q.sizes() && v.sizes() == q.sizes(),
                    "q/k/v/out must share shape");
  const auto dt = q.scalar_type();
  TORCH_CHECK_VALUE((dt == at::kBFloat16 || dt == at::kHalf) && k.scalar_type() == dt && v.scalar_type() == dt &&
                        out.scalar_type() == dt,
                    "q/k/v/out must share one dtype, bf16 or fp16");
  TORCH_CHECK_VALUE(beta.scalar_type() == at::kFloat || beta.scalar_type() == at::kBFloat16,
                    "beta must be fp32 or bf16");
  TORCH_CHECK_VALUE(g.numel() == n * t * h && beta.numel() == n * t * h, "g and beta must hold N*t*H values");
  for (const at::Tensor* x : {&q, &k, &v, &g, &beta, (const at::Tensor*)&state, (const at::Tensor*)&out})
    TORCH_CHECK_VALUE(x->is_contiguous(), "recurrent operands must be contiguous (the state is updated in place)");
  const at::Tensor gf = g.scalar_type() == at::kFloat ? g : g.to(at::kFloat);
  const int dtype_flags = (beta.scalar_type() == at::kBFloat16 ? CQGDN_RECURRENT_BETA_BF16 : 0) |
                          (dt == at::kHalf ? CQGDN_RECURRENT_FP16 : 0);
  check(cqgdn_recurrent(cptr(q), cptr(k), cptr(v), gf.data_ptr<float>(), cptr(beta), dtype_flags,
                        state.data_ptr<float>(), mptr(out), (int)n, (int)t, (int)h, (float)scale, stream_of(q)),
        "cqgdn_recurrent");
}

// models/decoding.py:16-78 between the projection and out_proj: proj [N,2,P] bf16 (P = (2 HK + 2 H) * 128 + 2 H),
// conv history bf16 [N,K-1,C] (C = (2 HK + H) * 128) and state fp32 [N,H,V,K] updated in place.
at::Tensor layer_decode_step(const at::Tensor& proj, const at::Tensor& conv_w, const at::Tensor& A_log,
                             const at::Tensor& dt_bias, const at::Tensor& norm_w, at::Tensor& history,
                             at::Tensor& state, int64_t heads, int64_t key_heads, double eps, double scale) {
  for (const at::Tensor* x : {&proj, &conv_w, &A_log, &dt_bias, &norm_w, (const at::Tensor*)&history,
                              (const at::Tensor*)&state})
    TORCH_CHECK_VALUE(on_gpu(*x), "the hip GDN backend requires tensors on a ROCm GPU");
  auto ok_heads = [](int64_t x) { return x == 4 || x == 8 || x == 16 || x == 32; };
  TORCH_CHECK_VALUE(ok_heads(heads) && ok_heads(key_heads) && heads % key_heads == 0, "heads=", heads,
                    ", key_heads=", key_heads, ": supported are 4, 8, 16, 32, key heads dividing heads");
  const int64_t C = (2 * key_heads + heads) * CQGDN_HEAD_DIM, width = C + heads * CQGDN_HEAD_DIM + 2 * heads;
  TORCH_CHECK_VALUE(proj.dim() == 3 && proj.size(1) == 2 && proj.size(2) == width &&
                        proj.scalar_type() == at::kBFloat16,
                    "proj must be bf16 [N, 2, (2*key_heads + 2*heads)*128 + 2*heads]");
  const int64_t N = proj.size(0), K = conv_w.dim() == 2 ? conv_w.size(1) : 0;
  TORCH_CHECK_VALUE(conv_w.dim() == 2 && conv_w.size(0) == C && conv_w.scalar_type() == at::kBFloat16,
                    "conv_weight must be bf16 [(2*key_heads + heads)*128, K]");
  TORCH_CHECK_VALUE(history.sizes() == at::IntArrayRef({N, K - 1, C}) && history.scalar_type() == at::kBFloat16 &&
                        history.is_contiguous(),
                    "cache['conv'] must be contiguous bf16 [N, K-1, (2*key_heads + heads)*128]");
  TORCH_CHECK_VALUE(state.sizes() == at::IntArrayRef({N, heads, 128, 128}) && state.scalar_type() == at::kFloat &&
                        state.is_contiguous(),
                    "cache['state'] must be contiguous fp32 [N, H, 128, 128] (value-first)");
  TORCH_CHECK_VALUE(A_log.numel() == heads && dt_bias.numel() == heads && norm_w.numel() == CQGDN_HEAD_DIM,
                    "A_log and dt_bias must hold H values, norm_weight 128");
  const at::Tensor p = proj.contiguous(), w = conv_w.contiguous();
  const at::Tensor alog = A_log.to(at::kFloat).contiguous(), dtb = dt_bias.to(at::kFloat).contiguous(),
                   nw = norm_w.to(at::kFloat).contiguous();
  at::Tensor out = at::empty({N, 2, heads * CQGDN_HEAD_DIM}, proj.options());
  check(cqgdn_layer_decode_step((int)N, (int)heads, (int)key_heads, (int)K, cptr(p), width, mptr(history), cptr(w),
                                alog.data_ptr<float>(), dtb.data_ptr<float>(), nw.data_ptr<float>(), (float)eps,
                                (float)scale, state.data_ptr<float>(), mptr(out), nullptr, 0, stream_of(proj)),
        "cqgdn_layer_decode_step");
  return out;
}

}  // namespace

TORCH_LIBRARY(cqgdn, m) {
  m.def("fwd(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor table, Tensor doc, float scale, int flags, "
        "Tensor? initial_state, bool want_state) -> (Tensor, Tensor, Tensor)");
  m.def("bwd(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor dy, Tensor table, Tensor doc, float scale, "
        "int flags, Tensor? ws) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("recurrent(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor(a!) state, Tensor(b!) out, "
        "float scale) -> ()");
  m.def("layer_decode_step(Tensor proj, Tensor conv_w, Tensor A_log, Tensor dt_bias, Tensor norm_w, "
        "Tensor(a!) history, Tensor(b!) state, int heads, int key_heads, float eps, float scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(cqgdn, CUDA, m) {
  m.impl("fwd", &fwd);
  m.impl("bwd", &bwd);
  m.impl("recurrent", &recurrent);
  m.impl("layer_decode_step", &layer_decode_step);
}

// CPU tensors reach the same functions only to be rejected: their first check raises the
// reference's ValueError for tensors off the GPU (ops/gated_delta_net.py raises before any launch).
TORCH_LIBRARY_IMPL(cqgdn, CPU, m) {
  m.impl("recurrent", &recurrent);
  m.impl("layer_decode_step", &layer_decode_step);
}
