// fw_radix_cuda -- PyTorch extension with the op names, signatures and outputs of the reference
// extension (src/cuda/binding.cpp:3-13, setup.py:5-8), implemented over the C ABI of libfwloss
// (include/fwloss.h).  This file holds no device code: it checks arguments, allocates outputs with
// the torch allocator, passes the current HIP stream and turns a non-zero status into a
// RuntimeError.
//
// Differences from the reference host code (src/cuda/fw_radix_argmax.cu:1381-1609), all additive:
//   * targets, kappas, masks and candidate tensors are validated (the reference checks only the
//     logits of the forwards, :1383-1386, :1419-1421);
//   * non-contiguous inputs are made contiguous instead of being read with the wrong strides (the
//     fused op reads rows of logits in place at any row stride);
//   * launches go on the current stream instead of the legacy default stream;
//   * any K is accepted by every op (the reference's small kernel has no bound check above
//     K = 10000, :1405-1408).
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "fwloss.h"

namespace {

hipStream_t current_stream(const at::Tensor& t) {
  return reinterpret_cast<hipStream_t>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

void check_status(int rc, const char* op) {
  TORCH_CHECK(rc == FWL_OK, op, ": ", fwl_status_string(rc));
}

// One workspace per (device, stream): calls on one stream are ordered, so they never use a
// workspace concurrently, and the library keeps no state in it from one call to the next.  A
// workspace that has to grow is replaced, but the superseded ones stay allocated until the process
// ends: a HIP graph captured on the stream keeps the device address it captured, and its replays
// must not write into memory the caching allocator has handed to another tensor since.  Growth is
// geometric, so the superseded ones add up to less than the current one.
at::Tensor workspace(const at::Tensor& like, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::vector<at::Tensor>> cache;
  const auto key = std::make_pair((int)like.get_device(), current_stream(like));
  std::lock_guard<std::mutex> lock(mu);
  std::vector<at::Tensor>& held = cache[key];
  if (held.empty() || (size_t)held.back().numel() < bytes) {
    size_t grow = bytes < 65536 ? 65536 : bytes;
    if (!held.empty() && grow < 2 * (size_t)held.back().numel()) grow = 2 * (size_t)held.back().numel();
    held.push_back(at::empty({(int64_t)grow}, like.options().dtype(at::kByte)));
  }
  return held.back();
}

void check_logits(const at::Tensor& logits) {
  // messages as in src/cuda/fw_radix_argmax.cu:1383-1386
  TORCH_CHECK(logits.is_cuda(), "logits must be a CUDA tensor");
  TORCH_CHECK(logits.dim() == 2, "logits must have shape [N, K]");
  TORCH_CHECK(logits.scalar_type() == torch::kFloat32, "logits must be float32");
  TORCH_CHECK(logits.size(1) >= 1, "logits must have K >= 1 classes");
}

void check_rows(const at::Tensor& t, const at::Tensor& logits, at::ScalarType dt, const char* name) {
  TORCH_CHECK(t.device() == logits.device(), name, " must be on the same device as logits");
  TORCH_CHECK(t.dim() == 1 && t.size(0) == logits.size(0), name, " must have shape [N]");
  TORCH_CHECK(t.scalar_type() == dt, name, " must be ", c10::toString(dt));
}

void check_matrix(const at::Tensor& t, const at::Tensor& logits, at::ScalarType dt, const char* name) {
  TORCH_CHECK(t.device() == logits.device(), name, " must be on the same device as logits");
  TORCH_CHECK(t.dim() == 2 && t.size(0) == logits.size(0) && t.size(1) == logits.size(1), name,
              " must have the shape of logits [N, K]");
  TORCH_CHECK(t.scalar_type() == dt, name, " must be ", c10::toString(dt));
}

struct Common {
  at::Tensor logits, targets, H, losses, mean, kappa, ws;
};

// element type of 16-bit or fp32 logits for the typed entry points
int fwl_dtype_of(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return FWL_FLOAT32;
    case torch::kBFloat16: return FWL_BFLOAT16;
    case torch::kFloat16: return FWL_FLOAT16;
    default: TORCH_CHECK(false, "logits must be float32, bfloat16 or float16");
  }
  return -1;
}

// checks, contiguous copies and the fp32/int32 per-row outputs; the reference ops take fp32
// logits only, the fused op also 16-bit ones
Common prepare(const at::Tensor& logits_in, const at::Tensor& targets_in, bool any_float = false) {
  if (any_float) {
    TORCH_CHECK(logits_in.is_cuda(), "logits must be a CUDA tensor");
    TORCH_CHECK(logits_in.dim() == 2, "logits must have shape [N, K]");
    fwl_dtype_of(logits_in);
    TORCH_CHECK(logits_in.size(1) >= 1, "logits must have K >= 1 classes");
  } else {
    check_logits(logits_in);
  }
  check_rows(targets_in, logits_in, torch::kInt64, "targets");
  Common c;
  c.logits = logits_in.contiguous();
  c.targets = targets_in.contiguous();
  const int64_t N = c.logits.size(0), K = c.logits.size(1);
  const auto f32 = c.logits.options().dtype(torch::kFloat32);
  c.H = torch::empty({N}, f32);
  c.losses = torch::empty({N}, f32);
  c.mean = torch::empty({}, f32);
  c.kappa = torch::empty({N}, c.logits.options().dtype(torch::kInt32));
  c.ws = workspace(c.logits, fwl_workspace_bytes(N, K));
  return c;
}

// fw_forward_small(logits, targets) -> [H, losses, mean_loss, kappa, selected_logits]
// (src/cuda/fw_radix_argmax.cu:1381-1414)
std::vector<at::Tensor> fw_forward_small(at::Tensor logits, at::Tensor targets) {
  c10::DeviceGuard guard(logits.device());
  Common c = prepare(logits, targets);
  const int64_t N = c.logits.size(0), K = c.logits.size(1);
  at::Tensor selected = torch::empty({N, K}, c.logits.options().dtype(torch::kBool));
  const int rc = fwl_forward_small(
      c.logits.data_ptr<float>(), c.targets.data_ptr<int64_t>(), N, K, c.H.data_ptr<float>(),
      c.losses.data_ptr<float>(), c.mean.data_ptr<float>(), c.kappa.data_ptr<int32_t>(),
      reinterpret_cast<uint8_t*>(selected.data_ptr<bool>()), c.ws.data_ptr(), (size_t)c.ws.numel(),
      current_stream(c.logits));
  check_status(rc, "fw_forward_small");
  return {c.H, c.losses, c.mean, c.kappa, selected};
}

// fw_backward_small(targets, selected_logits, kappas) -> grad   (:1591-1609)
at::Tensor fw_backward_small(at::Tensor targets, at::Tensor selected_logits, at::Tensor kappas) {
  TORCH_CHECK(selected_logits.is_cuda(), "selected_logits must be a CUDA tensor");
  TORCH_CHECK(selected_logits.dim() == 2, "selected_logits must have shape [N, K]");
  TORCH_CHECK(selected_logits.scalar_type() == torch::kBool, "selected_logits must be bool");
  c10::DeviceGuard guard(selected_logits.device());
  check_rows(targets, selected_logits, torch::kInt64, "targets");
  check_rows(kappas, selected_logits, torch::kInt32, "kappas");
  at::Tensor sel = selected_logits.contiguous(), tg = targets.contiguous(), kp = kappas.contiguous();
  const int64_t N = sel.size(0), K = sel.size(1);
  at::Tensor grad = torch::empty({N, K}, sel.options().dtype(torch::kFloat32));
  const int rc = fwl_backward_small(tg.data_ptr<int64_t>(), reinterpret_cast<const uint8_t*>(sel.data_ptr<bool>()),
                                    kp.data_ptr<int32_t>(), N, K, grad.data_ptr<float>(), current_stream(sel));
  check_status(rc, "fw_backward_small");
  return grad;
}

// fw_forward(logits, targets) -> [H, losses, mean_loss, kappa, candidate_buffer,
//                                 candidate_indices, candidate_counts]   (:1417-1496)
std::vector<at::Tensor> fw_forward(at::Tensor logits, at::Tensor targets) {
  c10::DeviceGuard guard(logits.device());
  Common c = prepare(logits, targets);
  const int64_t N = c.logits.size(0), K = c.logits.size(1);
  at::Tensor cbuf = torch::empty({N, K}, c.logits.options());
  at::Tensor cidx = torch::empty({N, K}, c.logits.options().dtype(torch::kInt32));
  at::Tensor ccnt = torch::empty({N}, c.logits.options().dtype(torch::kInt32));
  const int rc = fwl_forward_large(
      c.logits.data_ptr<float>(), c.targets.data_ptr<int64_t>(), N, K, c.H.data_ptr<float>(),
      c.losses.data_ptr<float>(), c.mean.data_ptr<float>(), c.kappa.data_ptr<int32_t>(),
      cbuf.data_ptr<float>(), cidx.data_ptr<int32_t>(), ccnt.data_ptr<int32_t>(), c.ws.data_ptr(),
      (size_t)c.ws.numel(), current_stream(c.logits));
  check_status(rc, "fw_forward");
  return {c.H, c.losses, c.mean, c.kappa, cbuf, cidx, ccnt};
}

// fw_backward(logits, targets, H, kappas, candidate_buffer, candidate_indices, candidate_counts)
// -> grad   (:1536-1559)
at::Tensor fw_backward(at::Tensor logits, at::Tensor targets, at::Tensor H, at::Tensor kappas,
                       at::Tensor candidate_buffer, at::Tensor candidate_indices,
                       at::Tensor candidate_counts) {
  check_logits(logits);
  c10::DeviceGuard guard(logits.device());
  check_rows(targets, logits, torch::kInt64, "targets");
  check_rows(H, logits, torch::kFloat32, "H");
  check_rows(kappas, logits, torch::kInt32, "kappas");
  check_matrix(candidate_buffer, logits, torch::kFloat32, "candidate_buffer");
  check_matrix(candidate_indices, logits, torch::kInt32, "candidate_indices");
  check_rows(candidate_counts, logits, torch::kInt32, "candidate_counts");
  at::Tensor z = logits.contiguous(), tg = targets.contiguous(), h = H.contiguous(), kp = kappas.contiguous(),
             cb = candidate_buffer.contiguous(), ci = candidate_indices.contiguous(),
             cc = candidate_counts.contiguous();
  const int64_t N = z.size(0), K = z.size(1);
  at::Tensor grad = torch::empty({N, K}, z.options());
  const int rc = fwl_backward_large(z.data_ptr<float>(), tg.data_ptr<int64_t>(), h.data_ptr<float>(),
                                    kp.data_ptr<int32_t>(), cb.data_ptr<float>(), ci.data_ptr<int32_t>(),
                                    cc.data_ptr<int32_t>(), N, K, grad.data_ptr<float>(), current_stream(z));
  check_status(rc, "fw_backward");
  return grad;
}

// fw_forward_backward(logits, targets, scale=1/N, reduce_div=N, path=-1, cand_cap=-1, losses64=False)
//   -> [H, losses, reduced, kappa, grad] (+ [losses64] when asked)
// The fused hot path: one launch, logits read once, dense gradient written once.  Logits may be
// float32, bfloat16 or float16 (grad has the logits' dtype, H, losses and reduced are float32) or
// float64 (every output fp64, as the reference CPU path computes them).  Rows of logits may lie any
// distance apart (a column slice such as logits[:, 1:] is read in place; grad is contiguous).
// path/cand_cap >= 0 set this call's dispatch switches (fwl_options); -1 keeps set_params's.
// losses64: also the fp64 per-row losses, the dtype of the reference's fw_loss_grad
// (src/cpu/fw_cpu.cpp:750-757).
std::vector<at::Tensor> fw_forward_backward(at::Tensor logits, at::Tensor targets, double scale, double reduce_div,
                                            int64_t path, int64_t cand_cap, bool losses64) {
  c10::DeviceGuard guard(logits.device());
  if (logits.is_cuda() && logits.dim() == 2 && logits.scalar_type() == torch::kFloat64) {
    // fp64 logits (the reference CPU path's other dtype): fp64 H, losses, reduced and grad
    TORCH_CHECK(logits.size(1) >= 1, "logits must have K >= 1 classes");
    check_rows(targets, logits, torch::kInt64, "targets");
    at::Tensor z = logits.contiguous(), y = targets.contiguous();
    const int64_t N = z.size(0), K = z.size(1);
    if (scale < 0) scale = N > 0 ? 1.0 / (double)N : 1.0;
    if (reduce_div < 0) reduce_div = (double)N;
    const auto f64 = z.options();
    at::Tensor H = torch::empty({N}, f64), losses = torch::empty({N}, f64), mean = torch::empty({}, f64);
    at::Tensor kappa = torch::empty({N}, z.options().dtype(torch::kInt32)), grad = torch::empty({N, K}, f64);
    check_status(fwl_forward_backward_f64(z.data_ptr<double>(), y.data_ptr<int64_t>(), N, K, scale, reduce_div,
                                          H.data_ptr<double>(), losses.data_ptr<double>(), mean.data_ptr<double>(),
                                          kappa.data_ptr<int32_t>(), grad.data_ptr<double>(), current_stream(z)),
                 "fw_forward_backward");
    if (losses64) return {H, losses, mean, kappa, grad, losses};
    return {H, losses, mean, kappa, grad};
  }
  TORCH_CHECK(logits.is_cuda(), "logits must be a CUDA tensor");
  TORCH_CHECK(logits.dim() == 2, "logits must have shape [N, K]");
  const int dtype = fwl_dtype_of(logits);
  TORCH_CHECK(logits.size(1) >= 1, "logits must have K >= 1 classes");
  check_rows(targets, logits, torch::kInt64, "targets");
  // rows in place when their elements are adjacent; anything else is copied
  at::Tensor z = logits;
  if (z.size(0) > 1 ? !(z.stride(1) == 1 && z.stride(0) >= z.size(1)) : z.stride(1) != 1) z = z.contiguous();
  const int64_t N = z.size(0), K = z.size(1);
  const int64_t ld = N > 1 ? z.stride(0) : K;
  at::Tensor y = targets.contiguous();
  if (scale < 0) scale = N > 0 ? 1.0 / (double)N : 1.0;
  if (reduce_div < 0) reduce_div = (double)N;
  const auto f32 = z.options().dtype(torch::kFloat32);
  at::Tensor H = torch::empty({N}, f32), losses = torch::empty({N}, f32), mean = torch::empty({}, f32);
  at::Tensor kappa = torch::empty({N}, z.options().dtype(torch::kInt32));
  at::Tensor l64;
  if (losses64) l64 = torch::empty({N}, z.options().dtype(torch::kFloat64));
  at::Tensor grad = torch::empty({N, K}, z.options().memory_format(at::MemoryFormat::Contiguous));
  fwl_options opt;
  opt.path = 0;
  opt.cand_cap = 0;
  const bool own = path >= 0 || cand_cap >= 0;
  if (own) {
    int dp = 0, dc = 0;
    fwl_get_params(&dp, &dc);
    opt.path = path >= 0 ? (int)path : dp;
    opt.cand_cap = cand_cap >= 0 ? (int)cand_cap : dc;
  }
  const size_t ws_bytes = fwl_workspace_bytes_ex(N, K, own ? &opt : nullptr);
  TORCH_CHECK(ws_bytes > 0, "fw_forward_backward: path must be in [0, 8] and cand_cap in [64, 512]");
  at::Tensor ws = workspace(z, ws_bytes);
  const int rc = fwl_forward_backward_ex(dtype, z.data_ptr(), ld, y.data_ptr<int64_t>(), N, K, scale, reduce_div,
                                         H.data_ptr<float>(), losses.data_ptr<float>(),
                                         losses64 ? l64.data_ptr<double>() : nullptr, mean.data_ptr<float>(),
                                         kappa.data_ptr<int32_t>(), grad.data_ptr(), ws.data_ptr(),
                                         (size_t)ws.numel(), own ? &opt : nullptr, current_stream(z));
  check_status(rc, "fw_forward_backward");
  if (losses64) return {H, losses, mean, kappa, grad, l64};
  return {H, losses, mean, kappa, grad};
}

// grad *= grad_output (a 0-dim factor, or one factor per row), in place; rows whose factor is 1
// are skipped on the device (src/cpu/fw_cpu.cpp:734-740)
at::Tensor fw_scale_grad(at::Tensor grad, at::Tensor grad_output) {
  TORCH_CHECK(grad.is_cuda() && grad.dim() == 2 && grad.is_contiguous(),
              "grad must be a contiguous CUDA tensor [N, K]");
  c10::DeviceGuard guard(grad.device());
  TORCH_CHECK(grad_output.device() == grad.device(), "grad_output must be on the device of grad");
  if (grad.scalar_type() == torch::kFloat64) {
    at::Tensor go = grad_output.to(torch::kFloat64).contiguous();
    TORCH_CHECK(go.numel() == 1 || (go.dim() == 1 && go.size(0) == grad.size(0)),
                "grad_output must be a scalar or have shape [N]");
    check_status(fwl_scale_grad_f64(grad.data_ptr<double>(), go.data_ptr<double>(), go.numel() == 1 ? 0 : 1,
                                    grad.size(0), grad.size(1), current_stream(grad)),
                 "fw_scale_grad");
    return grad;
  }
  const int dtype = fwl_dtype_of(grad);
  at::Tensor go = grad_output.to(torch::kFloat32).contiguous();
  int64_t stride = 0;
  if (go.numel() == 1) stride = 0;
  else {
    TORCH_CHECK(go.dim() == 1 && go.size(0) == grad.size(0), "grad_output must be a scalar or have shape [N]");
    stride = 1;
  }
  const int rc = fwl_scale_grad_typed(dtype, grad.data_ptr(), go.data_ptr<float>(), stride, grad.size(0),
                                      grad.size(1), current_stream(grad));
  check_status(rc, "fw_scale_grad");
  return grad;
}

// ---- the linear layer fused with the loss (logits = hidden @ weight^T, one vocabulary chunk at a
// time; no counterpart in the reference, whose ops take materialised logits)

// per-row state for a batch of N rows, initialised
at::Tensor fw_linear_state(at::Tensor like, int64_t N) {
  TORCH_CHECK(like.is_cuda(), "fw_linear_state: like must be a CUDA tensor");
  c10::DeviceGuard guard(like.device());
  at::Tensor st = torch::empty({(int64_t)fwl_linear_state_bytes(N) + 16}, like.options().dtype(torch::kUInt8));
  check_status(fwl_linear_begin(st.data_ptr(), N, current_stream(like)), "fw_linear_state");
  return st;
}

// merge the chunk logits [N, Vc] (columns v0 .. v0 + Vc - 1) into the state
void fw_linear_chunk(at::Tensor state, at::Tensor logits, at::Tensor targets, int64_t v0, int64_t V) {
  TORCH_CHECK(logits.is_cuda() && logits.dim() == 2, "logits chunk must be a CUDA tensor [N, Vc]");
  c10::DeviceGuard guard(logits.device());
  check_rows(targets, logits, torch::kInt64, "targets");
  TORCH_CHECK(state.device() == logits.device() && state.scalar_type() == torch::kUInt8 &&
                  (size_t)state.numel() >= fwl_linear_state_bytes(logits.size(0)),
              "state must come from fw_linear_state for these rows");
  at::Tensor z = logits.stride(1) == 1 ? logits : logits.contiguous();
  at::Tensor y = targets.contiguous();
  check_status(fwl_linear_chunk(fwl_dtype_of(z), z.data_ptr(), z.size(0), z.size(1), z.stride(0), v0, V,
                                y.data_ptr<int64_t>(), state.data_ptr(), current_stream(z)),
               "fw_linear_chunk");
}

// [H, losses, kappa, support [N, cap] int32, overflow [N] int32] after the last chunk
std::vector<at::Tensor> fw_linear_finish(at::Tensor state, at::Tensor targets, int64_t V) {
  TORCH_CHECK(targets.is_cuda() && targets.dim() == 1 && targets.scalar_type() == torch::kInt64,
              "targets must be a CUDA int64 tensor [N]");
  c10::DeviceGuard guard(targets.device());
  const int64_t N = targets.size(0);
  TORCH_CHECK(state.device() == targets.device() && state.scalar_type() == torch::kUInt8 &&
                  (size_t)state.numel() >= fwl_linear_state_bytes(N),
              "state must come from fw_linear_state for these rows");
  at::Tensor y = targets.contiguous();
  const auto f32 = y.options().dtype(torch::kFloat32), i32 = y.options().dtype(torch::kInt32);
  at::Tensor H = torch::empty({N}, f32), losses = torch::empty({N}, f32), kappa = torch::empty({N}, i32);
  at::Tensor support = torch::empty({N, (int64_t)fwl_linear_support_cap()}, i32);
  at::Tensor overflow = torch::empty({N}, i32);
  check_status(fwl_linear_finish(state.data_ptr(), y.data_ptr<int64_t>(), N, V, H.data_ptr<float>(),
                                 losses.data_ptr<float>(), kappa.data_ptr<int32_t>(), support.data_ptr<int32_t>(),
                                 overflow.data_ptr<int32_t>(), current_stream(y)),
               "fw_linear_finish");
  return {H, losses, kappa, support, overflow};
}

// [dhidden, dweight] of the rows with kappa > 0 (rows with kappa 0 contribute nothing), for the
// gradient with per-row scale row_scale (one value, or one per row)
std::vector<at::Tensor> fw_linear_grads(at::Tensor hidden, at::Tensor weight, at::Tensor targets, at::Tensor kappa,
                                        at::Tensor support, at::Tensor row_scale, bool want_dh, bool want_dw) {
  TORCH_CHECK(hidden.is_cuda() && hidden.dim() == 2 && weight.dim() == 2 && hidden.size(1) == weight.size(1),
              "hidden [N, d] and weight [V, d] must be CUDA tensors with the same d");
  TORCH_CHECK(hidden.scalar_type() == weight.scalar_type(), "hidden and weight must have one dtype");
  c10::DeviceGuard guard(hidden.device());
  const int64_t N = hidden.size(0), d = hidden.size(1), V = weight.size(0);
  const int dt = fwl_dtype_of(hidden);
  at::Tensor h = hidden.contiguous(), w = weight.contiguous(), y = targets.contiguous();
  at::Tensor kap = kappa.contiguous(), sup = support.contiguous();
  TORCH_CHECK(y.size(0) == N && kap.size(0) == N && sup.size(0) == N &&
                  sup.size(1) == (int64_t)fwl_linear_support_cap() && kap.scalar_type() == torch::kInt32 &&
                  sup.scalar_type() == torch::kInt32,
              "targets, kappa and support must come from fw_linear_finish for these rows");
  at::Tensor rs = row_scale.to(torch::kFloat32).contiguous();
  TORCH_CHECK(rs.numel() == 1 || rs.numel() == N, "row_scale must have one value or one per row");
  const int64_t rs_stride = rs.numel() == 1 ? 0 : 1;
  const hipStream_t s = current_stream(h);
  at::Tensor dh, dW;
  if (want_dh) {
    dh = torch::zeros_like(h);
    check_status(fwl_linear_dhidden(dt, w.data_ptr(), V, d, y.data_ptr<int64_t>(), kap.data_ptr<int32_t>(),
                                    sup.data_ptr<int32_t>(), rs.data_ptr<float>(), rs_stride, N, dh.data_ptr(), s),
                 "fw_linear_grads (dhidden)");
  }
  if (want_dw) {
    dW = torch::zeros_like(w);
    // entries per row: the support, plus the label when it lies outside the support
    const int64_t cap = sup.size(1);
    at::Tensor live = kap > 0;
    at::Tensor pos = torch::arange(cap, kap.options()).unsqueeze(0) < kap.unsqueeze(1);
    at::Tensor lab_in = ((sup == y.unsqueeze(1).to(torch::kInt32)) & pos).any(1);
    at::Tensor lab_ok = (y >= 0) & (y < V);
    at::Tensor cnt = (kap.clamp_min(0).to(torch::kInt64) + (live & lab_ok & lab_in.logical_not()).to(torch::kInt64));
    at::Tensor incl = cnt.cumsum(0);
    at::Tensor offsets = incl - cnt;
    // The number of entries sizes the sort.  Eagerly it is read back (one wait for the device);
    // under HIP graph capture, where the host cannot wait, the key array has room for every row's
    // largest count instead, and the slots past the entries hold a key of column V, which sorts
    // last and dweight skips (measured at N = 8192, V = 128256: about 0.4 ms more per backward).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    TORCH_CHECK(hipStreamIsCapturing(s, &cs) == hipSuccess, "fw_linear_grads: hipStreamIsCapturing failed");
    const bool padded = cs != hipStreamCaptureStatusNone;
    const int64_t P = padded ? N * (cap + 1) : (N > 0 ? incl[N - 1].item<int64_t>() : 0);
    if (P > 0) {
      at::Tensor keys = padded ? torch::full({P}, V * 2 * N, y.options()) : torch::empty({P}, y.options());
      at::Tensor vals = padded ? torch::zeros({P}, y.options().dtype(torch::kFloat32))
                               : torch::empty({P}, y.options().dtype(torch::kFloat32));
      check_status(fwl_linear_coo(y.data_ptr<int64_t>(), N, V, kap.data_ptr<int32_t>(), sup.data_ptr<int32_t>(),
                                  offsets.data_ptr<int64_t>(), rs.data_ptr<float>(), rs_stride,
                                  keys.data_ptr<int64_t>(), vals.data_ptr<float>(), s),
                   "fw_linear_grads (entries)");
      auto sorted = keys.sort();
      at::Tensor skeys = std::get<0>(sorted).contiguous();
      at::Tensor svals = vals.index_select(0, std::get<1>(sorted)).contiguous();
      check_status(fwl_linear_dweight(dt, h.data_ptr(), N, V, d, skeys.data_ptr<int64_t>(), svals.data_ptr<float>(),
                                      P, dW.data_ptr(), s),
                   "fw_linear_grads (dweight)");
    }
  }
  return {dh, dW};
}

void set_params(int64_t path, int64_t cand_cap) {
  check_status(fwl_set_params((int)path, (int)cand_cap), "set_params");
}

std::pair<int64_t, int64_t> get_params() {
  int p = 0, c = 0;
  fwl_get_params(&p, &c);
  return {p, c};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("fw_forward", &fw_forward, "FW loss forward with candidate lists (MI355X)");
  m.def("fw_backward", &fw_backward, "FW loss backward from candidate lists (MI355X)");
  m.def("fw_forward_small", &fw_forward_small, "FW loss forward with the support mask (MI355X)");
  m.def("fw_backward_small", &fw_backward_small, "FW loss backward from the support mask (MI355X)");
  m.def("fw_forward_backward", &fw_forward_backward, "Fused FW loss forward + backward (MI355X)",
        py::arg("logits"), py::arg("targets"), py::arg("scale") = -1.0, py::arg("reduce_div") = -1.0,
        py::arg("path") = -1, py::arg("cand_cap") = -1, py::arg("losses64") = false);
  m.def("fw_linear_state", &fw_linear_state, "Per-row state of the linear layer fused with the loss");
  m.def("fw_linear_chunk", &fw_linear_chunk, "Merge one vocabulary chunk of logits into the state");
  m.def("fw_linear_finish", &fw_linear_finish, "H, losses, kappa, support columns and overflow flags");
  m.def("fw_linear_grads", &fw_linear_grads, "Sparse dhidden and dweight from the supports",
        py::arg("hidden"), py::arg("weight"), py::arg("targets"), py::arg("kappa"), py::arg("support"),
        py::arg("row_scale"), py::arg("want_dh") = true, py::arg("want_dw") = true);
  m.def("fw_scale_grad", &fw_scale_grad, "In-place grad *= grad_output (device-side skip when 1)");
  m.def("set_params", &set_params, "Default dispatch switches: path (0 auto, 1 wave registers, 2 block stream, "
        "3 block stream with the overflow solve forced, 4 wave stream, 5 wave stream with the overflow solve forced, "
        "6 short-row segments, 7 split rows, 8 = 1 without line-aligned windows), cand_cap",
        py::arg("path"), py::arg("cand_cap") = 512);
  m.def("get_params", &get_params);
}
