// Eager autograd node of the public APIs (sigmoid_attention,
// sigmoid_attention_padded, sigmoid_attention_varlen), in C++.
//
// The reference builds its eager path from torch.autograd.Function-style
// registrations in Python (src/triton_sigmoid/sigmoid_triton_dense.py:696-753,
// sigmoid_triton_padded.py:780-846).  The same node written in Python costs
// tens of microseconds of host time per forward+backward before any kernel
// runs -- more than a small problem's kernels take -- and PyTorch's autograd
// engine runs a CUDA node's backward on its device thread, where a Python
// node must take the GIL.  This module is that node in C++: the forward
// launches the library's forward on the canonical tensors the Python layer
// prepared and saves them; the backward launches the library's backward on
// them.  Launch policy is the Python layer's (_capi._launch_fwd,
// _capi._launch_bwd): the forward passes the workspace
// sigattn_fwd_workspace_bytes asks for; the backward takes the range-split
// recompute backward when a small grid splits, else the two-pass kernels at
// the head dims and workspace limit the Python layer configures (in head
// groups when the whole problem's dS does not fit, unless a group's
// dQ-from-dS grid would have fewer workgroups than the GPU has compute
// units), else the recompute backward.  Workspaces come from
// torch's caching allocator; a workspace that cannot be allocated falls back
// to the kernels that need none.
//
// The library's entry points arrive as addresses from the Python layer
// (bind()), so this module calls the very library _capi loaded.  No HIP
// kernels live here.

#include <torch/extension.h>

#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/sigattn.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

struct Api {
  decltype(&sigattn_strerror) strerror = nullptr;
  decltype(&sigattn_fwd_workspace_bytes) fwd_workspace_bytes = nullptr;
  decltype(&sigattn_fwd_ws) fwd_ws = nullptr;
  decltype(&sigattn_bwd_workspace_bytes) bwd_workspace_bytes = nullptr;
  decltype(&sigattn_bwd_ws) bwd_ws = nullptr;
  decltype(&sigattn_bwd_split_workspace_bytes) bwd_split_workspace_bytes = nullptr;
  decltype(&sigattn_bwd_split) bwd_split = nullptr;
};
Api g_api;
bool g_bound = false;
std::vector<int64_t> g_two_pass_dims;
int64_t g_dq_ds_rows = 0;

void check_rc(int rc, const char *what) {
  TORCH_CHECK(rc == SIGATTN_OK, what, " failed: ", g_api.strerror(rc), " (status ", rc, ")");
}

int32_t dtype_code(const Tensor &t) {
  switch (t.scalar_type()) {
    case at::kHalf: return SIGATTN_F16;
    case at::kBFloat16: return SIGATTN_BF16;
    case at::kFloat: return SIGATTN_F32;
    default: TORCH_CHECK(false, "unsupported dtype ", t.scalar_type());
  }
  return -1;
}

const void *ptr_or_null(const Tensor &t) { return t.defined() ? t.data_ptr() : nullptr; }

// The sequence layout: seq_lens (padded [B, T, H, D], or undefined for
// dense) or cu_seqlens (packed [rows, H, D], with the longest sequences).
struct Layout {
  Tensor slq, slk, cuq, cuk;
  int64_t max_q = 0, max_k = 0;
  bool packed() const { return cuq.defined(); }
};

// The problem over canonical tensors: Q/K/V contiguous, fp32 bias / scale /
// score_mod and int32 seq_lens / cu_seqlens on Q's device (or undefined).
sigattn_problem make_problem(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &bias,
                             const Tensor &score_mod, const Tensor &scale, const Layout &lay, bool causal) {
  sigattn_problem p;
  std::memset(&p, 0, sizeof(p));
  p.abi_version = SIGATTN_ABI_VERSION;
  p.dtype = dtype_code(q);
  if (lay.packed()) {
    // An axis with no rows has no valid positions whatever max_seqlen says.
    p.B = lay.cuq.numel() - 1;
    p.Tq = q.size(0) > 0 ? lay.max_q : 0;
    p.Tk = k.size(0) > 0 ? lay.max_k : 0;
    p.H = q.size(1);
    p.D = q.size(2);
    p.q_stride_t = q.stride(0);
    p.q_stride_h = q.stride(1);
    p.k_stride_t = k.stride(0);
    p.k_stride_h = k.stride(1);
    p.cu_seqlens_q = static_cast<const int32_t *>(lay.cuq.data_ptr());
    p.cu_seqlens_k = static_cast<const int32_t *>(lay.cuk.data_ptr());
    p.rows_q = q.size(0);
    p.rows_k = k.size(0);
  } else {
    p.B = q.size(0);
    p.Tq = q.size(1);
    p.Tk = k.size(1);
    p.H = q.size(2);
    p.D = q.size(3);
    p.q_stride_b = q.stride(0);
    p.q_stride_t = q.stride(1);
    p.q_stride_h = q.stride(2);
    p.k_stride_b = k.stride(0);
    p.k_stride_t = k.stride(1);
    p.k_stride_h = k.stride(2);
    p.seq_lens_q = static_cast<const int32_t *>(ptr_or_null(lay.slq));
    p.seq_lens_k = static_cast<const int32_t *>(ptr_or_null(lay.slk));
  }
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.bias = static_cast<const float *>(ptr_or_null(bias));
  p.scale = static_cast<const float *>(ptr_or_null(scale));
  p.score_mod = static_cast<const float *>(ptr_or_null(score_mod));
  p.causal = causal ? 1 : 0;
  return p;
}

int compute_units(int dev) {
  static std::atomic<int> cache[64];
  if (dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// A uint8 workspace of `bytes` from the caching allocator, or an undefined
// tensor when none is needed or the device cannot hold it.
Tensor workspace(int64_t bytes, const Tensor &like) {
  if (bytes <= 0) return Tensor();
  try {
    return at::empty({bytes}, like.options().dtype(at::kByte));
  } catch (const c10::OutOfMemoryError &) {
    return Tensor();
  }
}

// Mirror of _capi.bwd_workspace_bytes: the two-pass backward's workspace, 0
// for the recompute backward.
int64_t two_pass_bytes(const sigattn_problem &p, int64_t limit, int dev) {
  bool two_pass = false;
  for (int64_t d : g_two_pass_dims) two_pass |= d == p.D;
  if (!two_pass) return 0;
  const int64_t full = (int64_t)g_api.bwd_workspace_bytes(&p);
  if (full <= limit) return full;
  const int64_t per_head = full / p.H;
  const int64_t heads = limit / per_head;
  const int64_t grid = heads * p.B * ((p.Tq + g_dq_ds_rows - 1) / g_dq_ds_rows);
  if (heads == 0 || grid < compute_units(dev)) return 0;
  return heads * per_head;
}

struct SigattnNode : public torch::autograd::Function<SigattnNode> {
  static Tensor forward(AutogradContext *ctx, const Tensor &q, const Tensor &k, const Tensor &v,
                        const Tensor &bias, const std::optional<Tensor> &score_mod, const Tensor &scale,
                        const std::optional<Tensor> &seq_lens_q, const std::optional<Tensor> &seq_lens_k,
                        bool causal, int64_t bwd_limit, const std::optional<Tensor> &cu_seqlens_q,
                        const std::optional<Tensor> &cu_seqlens_k, int64_t max_seqlen_q, int64_t max_seqlen_k) {
    const Tensor sm = score_mod.value_or(Tensor());
    const Layout lay{seq_lens_q.value_or(Tensor()), seq_lens_k.value_or(Tensor()), cu_seqlens_q.value_or(Tensor()),
                     cu_seqlens_k.value_or(Tensor()), max_seqlen_q, max_seqlen_k};
    ctx->save_for_backward({q, k, v, bias, scale, sm, lay.slq, lay.slk, lay.cuq, lay.cuk});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["bwd_limit"] = bwd_limit;
    ctx->saved_data["max_seqlen_q"] = max_seqlen_q;
    ctx->saved_data["max_seqlen_k"] = max_seqlen_k;
    // Packed rows with no sequence at all (B = 0) are zeros.
    if (lay.packed() && lay.cuq.numel() == 1) return at::zeros_like(q);
    Tensor out = at::empty_like(q);
    if (out.numel() == 0) return out;
    const c10::DeviceGuard guard(q.device());
    const sigattn_problem p = make_problem(q, k, v, bias, sm, scale, lay, causal);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    const int64_t nbytes = (int64_t)g_api.fwd_workspace_bytes(&p);
    Tensor ws = nbytes > 0 ? at::empty({nbytes}, q.options().dtype(at::kByte)) : Tensor();
    check_rc(g_api.fwd_ws(&p, out.data_ptr(), ws.defined() ? ws.data_ptr() : nullptr, nbytes, stream),
             "sigattn_fwd");
    return out;
  }

  static tensor_list backward(AutogradContext *ctx, tensor_list grads) {
    const auto saved = ctx->get_saved_variables();
    const Tensor &q = saved[0], &k = saved[1], &v = saved[2], &bias = saved[3], &scale = saved[4],
                 &sm = saved[5];
    const Layout lay{saved[6], saved[7], saved[8], saved[9], ctx->saved_data["max_seqlen_q"].toInt(),
                     ctx->saved_data["max_seqlen_k"].toInt()};
    const bool causal = ctx->saved_data["causal"].toBool();
    const int64_t limit = ctx->saved_data["bwd_limit"].toInt();
    Tensor dout = grads[0];
    if (dout.scalar_type() != q.scalar_type() || dout.device() != q.device() || !dout.is_contiguous())
      dout = dout.to(q.device(), q.scalar_type()).contiguous();
    TORCH_CHECK(dout.sizes() == q.sizes(), "dO shape ", dout.sizes(), " != Q shape ", q.sizes());
    const bool no_seqs = lay.packed() && lay.cuq.numel() == 1;  // B = 0: every packed row is outside
    Tensor dq = no_seqs ? at::zeros_like(q) : at::empty_like(q);
    Tensor dk = no_seqs ? at::zeros_like(k) : at::empty_like(k);
    Tensor dv = no_seqs ? at::zeros_like(v) : at::empty_like(v);
    tensor_list result(14);
    result[0] = dq, result[1] = dk, result[2] = dv;  // none for bias, score_mod, ... (no gradient)
    if ((dq.numel() == 0 && dk.numel() == 0) || no_seqs) return result;
    const c10::DeviceGuard guard(q.device());
    const int dev = q.device().index();
    const sigattn_problem p = make_problem(q, k, v, bias, sm, scale, lay, causal);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
    bool two_pass = false;
    for (int64_t d : g_two_pass_dims) two_pass |= d == p.D;
    const int64_t split = (int64_t)g_api.bwd_split_workspace_bytes(&p);
    if (split > 0 || !two_pass) {
      const Tensor ws = workspace(split, q);
      check_rc(g_api.bwd_split(&p, dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                               ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0, stream),
               "sigattn_bwd_split");
      return result;
    }
    const Tensor ws = workspace(two_pass_bytes(p, limit, dev), q);
    check_rc(g_api.bwd_ws(&p, dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                          ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0, stream),
             "sigattn_bwd_ws");
    return result;
  }
};

Tensor attention(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &bias,
                 const std::optional<Tensor> &score_mod, const Tensor &scale,
                 const std::optional<Tensor> &seq_lens_q, const std::optional<Tensor> &seq_lens_k, bool causal,
                 int64_t bwd_limit, const std::optional<Tensor> &cu_seqlens_q,
                 const std::optional<Tensor> &cu_seqlens_k, int64_t max_seqlen_q, int64_t max_seqlen_k) {
  TORCH_CHECK(g_bound, "_sigattn_autograd: bind() was not called");
  TORCH_CHECK(cu_seqlens_q.has_value() == cu_seqlens_k.has_value(),
              "_sigattn_autograd: cu_seqlens_q and cu_seqlens_k go together");
  return SigattnNode::apply(q, k, v, bias, score_mod, scale, seq_lens_q, seq_lens_k, causal, bwd_limit,
                            cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k);
}

template <class F> void bind_one(F &dst, const py::dict &fns, const char *name) {
  TORCH_CHECK(fns.contains(name), "_sigattn_autograd.bind: missing ", name);
  dst = reinterpret_cast<F>(fns[name].cast<uintptr_t>());
}

void bind(const py::dict &fns, const std::vector<int64_t> &two_pass_dims, int64_t dq_ds_rows) {
  Api api;
  bind_one(api.strerror, fns, "sigattn_strerror");
  bind_one(api.fwd_workspace_bytes, fns, "sigattn_fwd_workspace_bytes");
  bind_one(api.fwd_ws, fns, "sigattn_fwd_ws");
  bind_one(api.bwd_workspace_bytes, fns, "sigattn_bwd_workspace_bytes");
  bind_one(api.bwd_ws, fns, "sigattn_bwd_ws");
  bind_one(api.bwd_split_workspace_bytes, fns, "sigattn_bwd_split_workspace_bytes");
  bind_one(api.bwd_split, fns, "sigattn_bwd_split");
  TORCH_CHECK(dq_ds_rows > 0, "_sigattn_autograd.bind: dq_ds_rows must be positive");
  g_api = api;
  g_two_pass_dims = two_pass_dims;
  g_dq_ds_rows = dq_ds_rows;
  g_bound = true;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "C++ autograd node of sigmoid_attention / sigmoid_attention_padded over libsigattn";
  m.def("bind", &bind, "Entry point addresses of libsigattn (name -> address), two-pass head dims, "
        "query rows per dQ-from-dS workgroup");
  m.def("attention", &attention,
        "Forward with autograd; arguments are the canonical tensors of _capi._prepare (and _prepare_packed "
        "for the packed layout, with the longest sequences)",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("bias"), py::arg("score_mod"), py::arg("scale"),
        py::arg("seq_lens_q"), py::arg("seq_lens_k"), py::arg("causal"), py::arg("bwd_limit"),
        py::arg("cu_seqlens_q") = py::none(), py::arg("cu_seqlens_k") = py::none(), py::arg("max_seqlen_q") = 0,
        py::arg("max_seqlen_k") = 0);
}
