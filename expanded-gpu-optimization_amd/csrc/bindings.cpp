// fused_hoad._C: the torch-facing boundary of the MI355X kernels.
//
// Same module name, functions, argument names, defaults, return order, check order and
// messages as /root/reference/csrc/bindings.cpp:9-66, so Python callers and their tests see
// the same API. Each call validates the tensors, allocates outputs (and the backward's
// workspace) with the torch caching allocator on the inputs' device, and enqueues the kernels
// on the current stream through the C ABI in include/fused_hoad.h. No host synchronization.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <array>
#include <vector>

#include "fused_hoad.h"
#include "mlp_abi.h"

namespace {

constexpr int64_t kParameterCount = 12737;

// Check order and messages follow /root/reference/csrc/bindings.cpp:9-24. PyTorch-ROCm
// tensors report device type "cuda", hence the CUDA wording.
void check_inputs(const torch::Tensor& coordinates, const torch::Tensor& parameters) {
  TORCH_CHECK(coordinates.is_cuda(), "coordinates must be a CUDA tensor");
  TORCH_CHECK(parameters.is_cuda(), "parameters must be a CUDA tensor");
  TORCH_CHECK(coordinates.is_contiguous(), "coordinates must be contiguous");
  TORCH_CHECK(parameters.is_contiguous(), "parameters must be contiguous");
  TORCH_CHECK(coordinates.scalar_type() == torch::kFloat32, "coordinates must use float32");
  TORCH_CHECK(parameters.scalar_type() == torch::kFloat32, "parameters must use float32");
  TORCH_CHECK(coordinates.dim() == 2 && coordinates.size(1) == 2,
              "coordinates must have shape [batch, 2]");
  TORCH_CHECK(parameters.dim() == 1 && parameters.numel() == kParameterCount,
              "parameters must have shape [12737]");
  TORCH_CHECK(coordinates.device() == parameters.device(),
              "coordinates and parameters must be on the same device");
}

void check_status(int status) {
  TORCH_CHECK(status == FHOAD_SUCCESS, "fused_hoad kernel error (", fhoad_status_string(status),
              "): ", fhoad_last_error());
}

void* current_stream(const torch::Tensor& tensor) {
  return static_cast<void*>(
      at::hip::getCurrentHIPStreamMasqueradingAsCUDA(tensor.get_device()).stream());
}

}  // namespace

std::vector<torch::Tensor> fused_forward_laplacian(torch::Tensor coordinates,
                                                   torch::Tensor parameters, int64_t version) {
  TORCH_CHECK(version >= 0 && version <= 5, "version must be 0 to 5");
  check_inputs(coordinates, parameters);
  const c10::DeviceGuard device_guard(coordinates.device());
  const int64_t batch = coordinates.size(0);
  auto output = torch::empty({batch, 1}, coordinates.options());
  auto laplacian = torch::empty({batch, 1}, coordinates.options());
  if (batch == 0) {
    return {output, laplacian};
  }
  check_status(fhoad_forward_laplacian(coordinates.data_ptr<float>(), parameters.data_ptr<float>(),
                                       output.data_ptr<float>(), laplacian.data_ptr<float>(),
                                       batch, static_cast<int>(version),
                                       current_stream(coordinates)));
  return {output, laplacian};
}

std::vector<torch::Tensor> fused_forward_laplacian_backward(torch::Tensor coordinates,
                                                            torch::Tensor parameters,
                                                            torch::Tensor grad_output,
                                                            torch::Tensor grad_laplacian,
                                                            int64_t version) {
  TORCH_CHECK(version >= 1 && version <= 6, "backward version must be 1 to 6");
  check_inputs(coordinates, parameters);
  for (const auto& grad : {grad_output, grad_laplacian}) {
    TORCH_CHECK(grad.is_cuda() && grad.is_contiguous() && grad.scalar_type() == torch::kFloat32,
                "upstream gradients must be contiguous float32 CUDA tensors");
    TORCH_CHECK(grad.numel() == coordinates.size(0), "upstream gradients must have [batch] values");
    TORCH_CHECK(grad.device() == coordinates.device(),
                "upstream gradients must be on the coordinates' device");
  }
  const c10::DeviceGuard device_guard(coordinates.device());
  const int64_t batch = coordinates.size(0);
  auto grad_coordinates = torch::empty_like(coordinates);
  if (batch == 0) {
    return {torch::zeros_like(parameters), grad_coordinates};
  }
  auto grad_parameters = torch::empty_like(parameters);
  const size_t workspace_bytes = fhoad_backward_workspace_size(batch);
  auto workspace = torch::empty({static_cast<int64_t>(workspace_bytes)},
                                coordinates.options().dtype(torch::kUInt8));
  check_status(fhoad_forward_laplacian_backward(
      coordinates.data_ptr<float>(), parameters.data_ptr<float>(), grad_output.data_ptr<float>(),
      grad_laplacian.data_ptr<float>(), grad_parameters.data_ptr<float>(),
      grad_coordinates.data_ptr<float>(), workspace.data_ptr(), workspace_bytes, batch,
      static_cast<int>(version), current_stream(coordinates)));
  return {grad_parameters, grad_coordinates};
}

// The forward of the autograd glue's "saved" mode: (u, Laplacian, saved layers), the last an
// opaque uint8 buffer of fhoad_saved_layers_size(batch) bytes for backward_for_autograd.
std::vector<torch::Tensor> forward_saving(torch::Tensor coordinates, torch::Tensor parameters,
                                          int64_t version) {
  TORCH_CHECK(version >= 0 && version <= 5, "version must be 0 to 5");
  check_inputs(coordinates, parameters);
  const c10::DeviceGuard device_guard(coordinates.device());
  const int64_t batch = coordinates.size(0);
  auto output = torch::empty({batch, 1}, coordinates.options());
  auto laplacian = torch::empty({batch, 1}, coordinates.options());
  const size_t saved_bytes = fhoad_saved_layers_size(batch);
  TORCH_CHECK(saved_bytes <= static_cast<size_t>(INT64_MAX),
              "the saved layers of ", batch, " points do not fit in memory");
  auto saved = torch::empty({static_cast<int64_t>(saved_bytes)},
                            coordinates.options().dtype(torch::kUInt8));
  if (batch == 0) {
    return {output, laplacian, saved};
  }
  check_status(fhoad_forward_laplacian_saving(
      coordinates.data_ptr<float>(), parameters.data_ptr<float>(), output.data_ptr<float>(),
      laplacian.data_ptr<float>(), saved.data_ptr(), saved_bytes, batch,
      static_cast<int>(version), current_stream(coordinates)));
  return {output, laplacian, saved};
}

// The backward for the autograd glue (no counterpart among the reference's bindings): either
// upstream gradient may be None (zero, so no zeros tensor is made), and grad_coordinates is
// computed only when want_coordinates is set (otherwise None is returned and nothing is
// written). Same checks and kernels as fused_forward_laplacian_backward. saved:
// forward_saving's buffer for the same coordinates and parameters (the backward then reads the
// hidden layers instead of re-running the forward), or None.
std::vector<c10::optional<torch::Tensor>> backward_for_autograd(
    torch::Tensor coordinates, torch::Tensor parameters, c10::optional<torch::Tensor> grad_output,
    c10::optional<torch::Tensor> grad_laplacian, bool want_coordinates, int64_t version,
    c10::optional<torch::Tensor> saved) {
  TORCH_CHECK(version >= 1 && version <= 6, "backward version must be 1 to 6");
  check_inputs(coordinates, parameters);
  if (saved.has_value()) {
    TORCH_CHECK(saved->is_cuda() && saved->is_contiguous() && saved->scalar_type() == torch::kUInt8,
                "saved layers must be a contiguous uint8 CUDA tensor");
    TORCH_CHECK(saved->device() == coordinates.device(),
                "saved layers must be on the coordinates' device");
    TORCH_CHECK(static_cast<size_t>(saved->numel()) >= fhoad_saved_layers_size(coordinates.size(0)),
                "saved layers do not cover the batch");
  }
  for (const auto* grad : {&grad_output, &grad_laplacian}) {
    if (!grad->has_value()) continue;
    const torch::Tensor& g = **grad;
    TORCH_CHECK(g.is_cuda() && g.is_contiguous() && g.scalar_type() == torch::kFloat32,
                "upstream gradients must be contiguous float32 CUDA tensors");
    TORCH_CHECK(g.numel() == coordinates.size(0), "upstream gradients must have [batch] values");
    TORCH_CHECK(g.device() == coordinates.device(),
                "upstream gradients must be on the coordinates' device");
  }
  const c10::DeviceGuard device_guard(coordinates.device());
  const int64_t batch = coordinates.size(0);
  c10::optional<torch::Tensor> grad_coordinates;
  if (want_coordinates) grad_coordinates = torch::empty_like(coordinates);
  if (batch == 0) {
    return {torch::zeros_like(parameters), grad_coordinates};
  }
  auto grad_parameters = torch::empty_like(parameters);
  const size_t workspace_bytes = fhoad_backward_workspace_size(batch);
  auto workspace = torch::empty({static_cast<int64_t>(workspace_bytes)},
                                coordinates.options().dtype(torch::kUInt8));
  const float* gu = grad_output.has_value() ? grad_output->data_ptr<float>() : nullptr;
  const float* gl = grad_laplacian.has_value() ? grad_laplacian->data_ptr<float>() : nullptr;
  float* gx = want_coordinates ? grad_coordinates->data_ptr<float>() : nullptr;
  if (saved.has_value()) {
    check_status(fhoad_forward_laplacian_backward_saved(
        coordinates.data_ptr<float>(), parameters.data_ptr<float>(), saved->data_ptr(),
        static_cast<size_t>(saved->numel()), gu, gl, grad_parameters.data_ptr<float>(), gx,
        workspace.data_ptr(), workspace_bytes, batch, static_cast<int>(version),
        current_stream(coordinates)));
  } else {
    check_status(fhoad_forward_laplacian_backward(
        coordinates.data_ptr<float>(), parameters.data_ptr<float>(), gu, gl,
        grad_parameters.data_ptr<float>(), gx, workspace.data_ptr(), workspace_bytes, batch,
        static_cast<int>(version), current_stream(coordinates)));
  }
  return {grad_parameters, grad_coordinates};
}

// Where each of the model's ten parameters sits in the packed buffer (mlp_abi.h), in layout
// order: weight then bias of each linear layer. cols == 0 marks a bias vector.
struct PackedSlice {
  int64_t offset, rows, cols;
};
constexpr int64_t hidden_base(int layer) { return fhoad::kHiddenBase + (layer - 1) * fhoad::kHiddenStride; }
constexpr std::array<PackedSlice, 10> kPackedSlices{{
    {0, fhoad::kHidden, fhoad::kInputs},
    {fhoad::kLayer0Bias, fhoad::kHidden, 0},
    {hidden_base(1), fhoad::kHidden, fhoad::kHidden},
    {hidden_base(1) + fhoad::kHidden * fhoad::kHidden, fhoad::kHidden, 0},
    {hidden_base(2), fhoad::kHidden, fhoad::kHidden},
    {hidden_base(2) + fhoad::kHidden * fhoad::kHidden, fhoad::kHidden, 0},
    {hidden_base(3), fhoad::kHidden, fhoad::kHidden},
    {hidden_base(3) + fhoad::kHidden * fhoad::kHidden, fhoad::kHidden, 0},
    {fhoad::kOutputBase, 1, fhoad::kHidden},
    {fhoad::kOutputBase + fhoad::kHidden, 1, 0},
}};
static_assert(fhoad::kOutputBase + fhoad::kHidden + 1 == kParameterCount, "packed slices");

// The autograd path of fused_laplacian's "cuda*" and "saved" modes as a C++ autograd Function:
// the same forward, backward and gradients as the Python Functions of fused.py, without their
// per-step host work (the Python apply, the backward's Python frame, the differentiable
// torch.cat pack and its backward, or the ten gradient views built in Python). Inputs:
// coordinates; the packed buffer when the model's parameters are its views
// (flatten_poisson_parameters_), else None; the forward and backward versions; whether to keep
// the hidden layers for the backward ("saved"); and the ten parameters in layout order (weight
// then bias of each linear layer), the Function's differentiable inputs. Without a buffer the
// parameters are packed into a new one (one copy kernel, outside autograd). Each parameter gets
// a view of the packed gradient with its own shape. An unused output's gradient arrives
// undefined and is read as zero; the coordinate gradient is computed only when the coordinates
// need it.
struct ModelLaplacian : public torch::autograd::Function<ModelLaplacian> {
  static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx,
                                                const torch::Tensor& coordinates,
                                                const c10::optional<torch::Tensor>& packed,
                                                int64_t version, int64_t backward_version,
                                                bool save_layers, torch::TensorList parameters) {
    TORCH_CHECK(backward_version >= 1 && backward_version <= 6, "backward version must be 1 to 6");
    TORCH_CHECK(parameters.size() == kPackedSlices.size(), "expected the model's 10 parameters");
    for (size_t k = 0; k < kPackedSlices.size(); ++k) {
      const PackedSlice& slice = kPackedSlices[k];
      const torch::Tensor& p = parameters[k];
      const bool shape_ok = slice.cols ? p.dim() == 2 && p.size(0) == slice.rows && p.size(1) == slice.cols
                                       : p.dim() == 1 && p.size(0) == slice.rows;
      TORCH_CHECK(shape_ok, "parameter ", k, " must have the shape of layout slice ", k);
    }
    torch::Tensor flat;
    if (packed.has_value()) {
      flat = *packed;
      check_inputs(coordinates, flat);
      const auto* base = static_cast<const char*>(flat.data_ptr());
      for (size_t k = 0; k < kPackedSlices.size(); ++k) {
        const torch::Tensor& p = parameters[k];
        TORCH_CHECK(p.is_contiguous() && static_cast<const char*>(p.data_ptr()) ==
                                             base + sizeof(float) * kPackedSlices[k].offset,
                    "parameter ", k, " is not the packed buffer's view at its layout offset");
      }
    } else {
      std::vector<torch::Tensor> pieces;
      pieces.reserve(parameters.size());
      for (const torch::Tensor& p : parameters) pieces.push_back(p.reshape({-1}));
      flat = torch::cat(pieces);
      check_inputs(coordinates, flat);
    }
    ctx->set_materialize_grads(false);
    ctx->saved_data["backward_version"] = backward_version;
    ctx->saved_data["packed_given"] = packed.has_value();
    ctx->saved_data["save_layers"] = save_layers;
    std::vector<torch::Tensor> out = save_layers ? forward_saving(coordinates, flat, version)
                                                 : fused_forward_laplacian(coordinates, flat, version);
    // Saved: coordinates, the packed buffer, the saved layers ("saved" mode) and, when the
    // buffer is the model's (its parameters are views of it), the ten parameters as well: each
    // view has its own version counter, so an in-place update of a parameter between this
    // forward and the backward (an optimizer step before a retain_graph backward) leaves the
    // buffer's counter alone; saving the views makes autograd's check of their counters raise
    // PyTorch's in-place-modification error there, as nn.Linear would. Saving copies nothing.
    std::vector<torch::Tensor> to_save{coordinates, flat};
    if (save_layers) to_save.push_back(out[2]);
    if (packed.has_value()) to_save.insert(to_save.end(), parameters.begin(), parameters.end());
    ctx->save_for_backward(to_save);
    return {out[0], out[1]};
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    // One gradient per forward argument: coordinates, packed, version, backward_version,
    // save_layers, then the ten parameters (undefined where none). The differentiable inputs
    // are the coordinates (input 0), the packed buffer when given, and the parameters.
    torch::autograd::variable_list result(5 + kPackedSlices.size());
    if (!grads[0].defined() && !grads[1].defined()) return result;
    const auto saved = ctx->get_saved_variables();
    const size_t first_parameter = ctx->saved_data["packed_given"].toBool() ? 2 : 1;
    const bool needs_coordinates = ctx->needs_input_grad(0);
    bool needs_parameters = false;
    for (size_t k = 0; k < kPackedSlices.size(); ++k) {
      needs_parameters |= ctx->needs_input_grad(first_parameter + k);
    }
    auto upstream = [](const torch::Tensor& g) -> c10::optional<torch::Tensor> {
      if (!g.defined()) return c10::nullopt;
      return g.reshape({-1}).contiguous();
    };
    const auto out = backward_for_autograd(
        saved[0], saved[1], upstream(grads[0]), upstream(grads[1]), needs_coordinates,
        ctx->saved_data["backward_version"].toInt(),
        ctx->saved_data["save_layers"].toBool() ? c10::optional<torch::Tensor>(saved[2])
                                                : c10::nullopt);
    if (needs_coordinates) result[0] = *out[1];
    if (needs_parameters) {
      const torch::Tensor& grad_flat = *out[0];
      for (size_t k = 0; k < kPackedSlices.size(); ++k) {
        if (!ctx->needs_input_grad(first_parameter + k)) continue;
        const PackedSlice& slice = kPackedSlices[k];
        result[5 + k] = slice.cols ? grad_flat.as_strided({slice.rows, slice.cols}, {slice.cols, 1}, slice.offset)
                                   : grad_flat.as_strided({slice.rows}, {1}, slice.offset);
      }
    }
    return result;
  }
};

torch::autograd::variable_list model_laplacian(const torch::Tensor& coordinates,
                                               const c10::optional<torch::Tensor>& packed,
                                               int64_t version, int64_t backward_version,
                                               bool save_layers,
                                               const std::vector<torch::Tensor>& parameters) {
  return ModelLaplacian::apply(coordinates, packed, version, backward_version, save_layers,
                               torch::TensorList(parameters));
}

// One fused Poisson PINN + Adam training step (fhoad_poisson_adam_step). No counterpart among
// the reference's bindings: it replaces the Python step of
// /root/reference/benchmarks/train_poisson.py:30-45 and benchmark_training.py:41-60 (fused
// forward, loss, fused backward, torch.optim.Adam). parameters, exp_avg, exp_avg_sq and step
// are updated in place; returns the loss (a 0-dim tensor) of the parameters on entry.
torch::Tensor poisson_adam_step(torch::Tensor coordinates, torch::Tensor source,
                                torch::Tensor parameters, torch::Tensor exp_avg,
                                torch::Tensor exp_avg_sq, torch::Tensor step, double lr,
                                double beta1, double beta2, double eps, double weight_decay,
                                c10::optional<torch::Tensor> grad_parameters,
                                c10::optional<torch::Tensor> grad_coordinates,
                                c10::optional<torch::Tensor> boundary, double boundary_weight) {
  check_inputs(coordinates, parameters);
  const int64_t batch = coordinates.size(0);
  TORCH_CHECK(batch > 0, "coordinates must hold at least one point");
  auto check_like = [&](const torch::Tensor& t, int64_t numel, const char* what) {
    TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.scalar_type() == torch::kFloat32, what,
                " must be a contiguous float32 CUDA tensor");
    TORCH_CHECK(t.numel() == numel, what, " must have ", numel, " values");
    TORCH_CHECK(t.device() == coordinates.device(), what, " must be on the coordinates' device");
  };
  check_like(source, batch, "source");
  check_like(exp_avg, kParameterCount, "exp_avg");
  check_like(exp_avg_sq, kParameterCount, "exp_avg_sq");
  check_like(step, 1, "step");
  float* grad_parameters_ptr = nullptr;
  float* grad_coordinates_ptr = nullptr;
  const float* boundary_ptr = nullptr;
  int64_t boundary_count = 0;
  if (grad_parameters.has_value()) {
    check_like(*grad_parameters, kParameterCount, "grad_parameters");
    grad_parameters_ptr = grad_parameters->data_ptr<float>();
  }
  if (grad_coordinates.has_value()) {
    check_like(*grad_coordinates, 2 * batch, "grad_coordinates");
    grad_coordinates_ptr = grad_coordinates->data_ptr<float>();
  }
  if (boundary.has_value()) {
    TORCH_CHECK(boundary->dim() == 2 && boundary->size(1) == 2,
                "boundary must have shape [count, 2]");
    boundary_count = boundary->size(0);
    check_like(*boundary, 2 * boundary_count, "boundary");
    boundary_ptr = boundary->data_ptr<float>();
  }
  TORCH_CHECK(boundary_weight >= 0.0, "boundary_weight must be non-negative");
  const c10::DeviceGuard device_guard(coordinates.device());
  auto loss = torch::empty({}, coordinates.options());
  const size_t workspace_bytes = fhoad_poisson_adam_step_workspace_size(batch, boundary_count);
  auto workspace = torch::empty({static_cast<int64_t>(workspace_bytes)},
                                coordinates.options().dtype(torch::kUInt8));
  check_status(fhoad_poisson_adam_step(
      coordinates.data_ptr<float>(), source.data_ptr<float>(), batch, boundary_ptr,
      boundary_count, boundary_weight, parameters.data_ptr<float>(), exp_avg.data_ptr<float>(),
      exp_avg_sq.data_ptr<float>(), step.data_ptr<float>(), loss.data_ptr<float>(),
      grad_parameters_ptr, grad_coordinates_ptr, workspace.data_ptr(), workspace_bytes, lr, beta1,
      beta2, eps, weight_decay, current_stream(coordinates)));
  return loss;
}

// Waits for the device's current stream and raises if a kernel since the last check gave up a
// bounded wait (fhoad_check_device).
void check_device(torch::Device device) {
  TORCH_CHECK(device.is_cuda(), "device must be a CUDA device");
  const c10::DeviceGuard device_guard(device);
  check_status(fhoad_check_device(static_cast<void*>(
      at::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index()).stream())));
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
  module.def("_check_device", &check_device,
             "Raise if a kernel on this device gave up a bounded wait since the last check",
             pybind11::arg("device"));
  module.def("poisson_adam_step", &poisson_adam_step,
             "Fused Poisson PINN training step with Adam on the packed parameters (MI355X)",
             pybind11::arg("coordinates"), pybind11::arg("source"), pybind11::arg("parameters"),
             pybind11::arg("exp_avg"), pybind11::arg("exp_avg_sq"), pybind11::arg("step"),
             pybind11::arg("lr"), pybind11::arg("beta1"), pybind11::arg("beta2"),
             pybind11::arg("eps"), pybind11::arg("weight_decay"),
             pybind11::arg("grad_parameters") = pybind11::none(),
             pybind11::arg("grad_coordinates") = pybind11::none(),
             pybind11::arg("boundary") = pybind11::none(),
             pybind11::arg("boundary_weight") = 100.0);
  module.def("_backward", &backward_for_autograd,
             "Backward for the autograd glue: optional upstream gradients (None is zero) and an "
             "optional coordinate gradient",
             pybind11::arg("coordinates"), pybind11::arg("parameters"),
             pybind11::arg("grad_output"), pybind11::arg("grad_laplacian"),
             pybind11::arg("want_coordinates"), pybind11::arg("version") = 6,
             pybind11::arg("saved") = pybind11::none());
  module.def("_model_laplacian", &model_laplacian,
             "(u, Laplacian) of the model's ten parameters through the C++ autograd Function",
             pybind11::arg("coordinates"), pybind11::arg("packed"), pybind11::arg("version"),
             pybind11::arg("backward_version"), pybind11::arg("save_layers"),
             pybind11::arg("parameters"));
  module.def("_forward_saving", &forward_saving,
             "Forward that also keeps the hidden layers' outputs for _backward(saved=...)",
             pybind11::arg("coordinates"), pybind11::arg("parameters"),
             pybind11::arg("version") = 2);
  module.def("fused_forward_laplacian", &fused_forward_laplacian,
             "Fixed MLP forward pass and input Laplacian (MI355X HIP kernel)",
             pybind11::arg("coordinates"), pybind11::arg("parameters"),
             pybind11::arg("version") = 2);
  module.def("fused_forward_laplacian_backward", &fused_forward_laplacian_backward,
             "Gradients of the fused forward Laplacian w.r.t. parameters and coordinates "
             "(MI355X HIP kernels)",
             pybind11::arg("coordinates"), pybind11::arg("parameters"),
             pybind11::arg("grad_output"), pybind11::arg("grad_laplacian"),
             pybind11::arg("version") = 6);
}
