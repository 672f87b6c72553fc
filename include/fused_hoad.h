/*
 * fused_hoad C ABI: the MI355X (gfx950) forward-Laplacian jet and adjoint-jet backward of
 * the fixed 2 -> 64 -> 64 -> 64 -> 64 -> 1 FP32 tanh MLP.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer to contiguous
 * float32 memory on the device that is current on the calling thread, and `stream` is a
 * hipStream_t (NULL = that device's default stream). Calls are asynchronous with respect to
 * the host: they enqueue work on `stream` and return. No call allocates device memory except
 * where stated; the backward takes its scratch as a caller-owned workspace.
 *
 * Parameters use the packed 12,737-float layout of the reference
 * (/root/reference/csrc/mlp_abi.cuh:8-17, src/fused_hoad/parameters.py:28-48):
 *   W0[64][2] @0, b0[64] @128, then for hidden layers 1..3: W[64][64] ([out][in]) and b[64]
 *   at 192 + 4160*(layer-1), then w_out[64] @12672 and b_out @12736.
 *
 * Every entry point returns FHOAD_SUCCESS (0) or an fhoad_status code; on failure
 * fhoad_last_error() returns a message for the calling thread.
 */
#ifndef FUSED_HOAD_H_
#define FUSED_HOAD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FHOAD_ABI_VERSION 1
#define FHOAD_PARAMETER_COUNT 12737

typedef enum fhoad_status {
  FHOAD_SUCCESS = 0,
  FHOAD_ERROR_INVALID_VERSION = 1,   /* version outside the accepted range */
  FHOAD_ERROR_INVALID_VALUE = 2,     /* null pointer or negative batch */
  FHOAD_ERROR_MISALIGNED = 3,        /* workspace not 16-byte aligned */
  FHOAD_ERROR_WORKSPACE = 4,         /* workspace missing or smaller than required */
  FHOAD_ERROR_DEVICE = 5             /* the HIP runtime reported an error */
} fhoad_status;

/* Version of this ABI (FHOAD_ABI_VERSION of the build). */
int fhoad_abi_version(void);

/* Number of floats in the packed parameter buffer: 12737 (mlp_abi.cuh:16-17). */
int64_t fhoad_parameter_count(void);

/* Static text for a status code. */
const char* fhoad_status_string(int status);

/* Message describing the last failed call on the calling thread ("" if none). */
const char* fhoad_last_error(void);

/*
 * Device-side failures that a launch cannot report: waits for `stream` to finish, then reads and
 * clears the status word of the current device. Returns FHOAD_ERROR_DEVICE with a message when
 * any kernel since the last check gave up a bounded wait: a forward's split tile (the tiles past
 * the last whole round, whose rows four waves share) waits for the other three waves at most
 * about 0.5 s per meeting, and a wave that gives up writes NaN for that tile's u and Laplacian
 * (and, in fhoad_forward_laplacian_saving, leaves that tile's saved layers undefined). Never
 * seen in tested runs; FHOAD_SUCCESS otherwise.
 *
 * No counterpart in the reference, whose kernels have no bounded waits; its launch errors
 * surface through C10_CUDA_KERNEL_LAUNCH_CHECK (/root/reference/csrc/fused_residual.cu:641),
 * as this library's do through each entry point's return code.
 */
int fhoad_check_device(void* stream);

/*
 * Forward Laplacian: output[b] = u(x_b) and laplacian[b] = (d2u/dx2 + d2u/dy2)(x_b) for
 * coordinates [batch][2] (x, y interleaved). output and laplacian each hold `batch` floats.
 * version 0..5 is accepted for API compatibility and every value runs the same gfx950
 * kernel. batch == 0 enqueues nothing.
 *
 * Replaces fused_forward_laplacian_cuda (/root/reference/csrc/fused_residual.cu:587-643),
 * which the pybind layer binds at /root/reference/csrc/bindings.cpp:28-36.
 */
int fhoad_forward_laplacian(const float* coordinates, const float* parameters, float* output,
                            float* laplacian, int64_t batch, int version, void* stream);

/*
 * Bytes of device workspace fhoad_forward_laplacian_backward needs for `batch` points: one
 * weight-gradient partial row of 12,800 floats per slot, at most 256 slots (13,107,200 bytes).
 * It depends only on the batch. 0 for batch <= 0.
 */
size_t fhoad_backward_workspace_size(int64_t batch);

/*
 * Backward of the forward Laplacian. Given dLoss/du (grad_output[batch]) and
 * dLoss/dLaplacian (grad_laplacian[batch]), writes dLoss/dparameters (grad_parameters[12737],
 * overwritten, not accumulated) and dLoss/dcoordinates (grad_coordinates[batch][2]).
 * grad_output or grad_laplacian may be NULL, meaning all zeros (a loss that uses only u or
 * only the Laplacian), and grad_coordinates may be NULL, meaning not written; the reference
 * requires all three. workspace must hold
 * fhoad_backward_workspace_size(batch) bytes and be 16-byte aligned (hipMalloc and torch
 * allocations are); its contents on entry are ignored. The
 * weight-gradient sum runs in a fixed order that does not depend on the grid size, so
 * results are bitwise reproducible. version 1..6 is accepted for API compatibility and every
 * value runs the same gfx950 kernels. batch == 0 zero-fills grad_parameters.
 *
 * Replaces fused_forward_laplacian_backward_cuda (/root/reference/csrc/fused_backward.cu:
 * 859-934), which the pybind layer binds at /root/reference/csrc/bindings.cpp:38-54.
 */
int fhoad_forward_laplacian_backward(const float* coordinates, const float* parameters,
                                     const float* grad_output, const float* grad_laplacian,
                                     float* grad_parameters, float* grad_coordinates,
                                     void* workspace, size_t workspace_bytes, int64_t batch,
                                     int version, void* stream);

/*
 * fhoad_forward_laplacian_backward without a workspace argument: it allocates nothing (no
 * hipMalloc, hipFree or allocating library call). Its scratch is a static device array inside
 * the library, one copy per GPU, held from the library's load on that GPU until the process
 * ends: 13,107,200 bytes (256 partial-row slots of 12,800 floats), the most the backward
 * needs for any batch, so every batch fits (a need beyond it would be rejected with
 * FHOAD_ERROR_WORKSPACE). Nothing in it has to start at zero. Every
 * call on one GPU shares that GPU's scratch, which keeps the last call's contents: calls that
 * overlap on one GPU (other streams, other host threads) race and must be serialized by the
 * caller. Results are bitwise those of fhoad_forward_laplacian_backward.
 *
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 */
int fhoad_forward_laplacian_backward_noalloc(const float* coordinates, const float* parameters,
                                             const float* grad_output, const float* grad_laplacian,
                                             float* grad_parameters, float* grad_coordinates,
                                             int64_t batch, int version, void* stream);

/*
 * Bytes of the saved-layer buffer fhoad_forward_laplacian_saving writes for `batch` points:
 * 49,152 bytes (the three hidden layers' outputs, 4 jet components x 64 neurons each) per
 * 16-point tile, ceil(batch / 16) tiles, i.e. 3 KB per point. 0 for batch <= 0; SIZE_MAX when
 * the size does not fit in size_t (no buffer can then be large enough).
 */
size_t fhoad_saved_layers_size(int64_t batch);

/*
 * fhoad_forward_laplacian that also writes the hidden layers' outputs (the forward jet after
 * each tanh) to `saved`, for fhoad_forward_laplacian_backward_saved. output and laplacian are
 * bitwise those of fhoad_forward_laplacian. saved must hold fhoad_saved_layers_size(batch)
 * bytes and be 16-byte aligned; its layout is private to this library.
 *
 * No counterpart in the reference, whose backward always re-runs the forward: it is for
 * autograd callers that can keep 3 KB per point between the forward and the backward.
 */
int fhoad_forward_laplacian_saving(const float* coordinates, const float* parameters,
                                   float* output, float* laplacian, void* saved,
                                   size_t saved_bytes, int64_t batch, int version, void* stream);

/*
 * fhoad_forward_laplacian_backward reading the hidden layers' outputs from `saved` (written by
 * fhoad_forward_laplacian_saving for the same coordinates and parameters, left unchanged since)
 * instead of re-running the forward: a third of the backward's matrix work. Same arguments,
 * contract and workspace as fhoad_forward_laplacian_backward, and bitwise the same results.
 * Batches of up to 12,288 points (the small-batch kernel) and the points past the last whole
 * round of 64-point tiles re-run the forward as before.
 *
 * No counterpart in the reference (see fhoad_forward_laplacian_saving).
 */
int fhoad_forward_laplacian_backward_saved(const float* coordinates, const float* parameters,
                                           const void* saved, size_t saved_bytes,
                                           const float* grad_output, const float* grad_laplacian,
                                           float* grad_parameters, float* grad_coordinates,
                                           void* workspace, size_t workspace_bytes, int64_t batch,
                                           int version, void* stream);

/*
 * Bytes of device workspace fhoad_poisson_adam_step needs for `batch` interior and
 * `boundary_count` boundary points. 0 for batch <= 0 or boundary_count < 0.
 */
size_t fhoad_poisson_adam_step_workspace_size(int64_t batch, int64_t boundary_count);

/*
 * One fused training step of the Poisson PINN loss with Adam:
 *   loss = mean_b (laplacian(x_b) - source[b])^2
 *          + boundary_weight * mean_k u(boundary_k)^2      (term absent when boundary_count == 0)
 * then one torch.optim.Adam update (amsgrad = False, maximize = False) of `parameters` in place.
 * Two kernels on `stream`:
 *   - the gradient kernel re-runs the forward jet, forms the residual (interior points) or u
 *     (boundary points) and the adjoint seed autograd would form for the loss in registers, and
 *     walks the adjoint back;
 *   - the reduction kernel sums the weight gradient in the backward's fixed order and applies
 *     Adam to each element in the same thread.
 * Arguments:
 *   coordinates, source: [batch][2] interior points and f[batch].
 *   boundary: [boundary_count][2] boundary points (NULL allowed when boundary_count == 0).
 *   parameters, exp_avg, exp_avg_sq: [12737] each, updated in place (Adam's first and second
 *     moments share the packed parameter layout).
 *   step: one float, the number of Adam steps taken so far; incremented on the device, so the
 *     call can be captured in a HIP graph and replayed.
 *   loss: one float, written with the loss of the parameters on entry.
 *   grad_parameters: optional [12737] copy of the summed gradient (NULL: not written).
 *   grad_coordinates: optional [batch][2] dLoss/d(interior coordinates) (NULL: not written).
 *   workspace: fhoad_poisson_adam_step_workspace_size(batch, boundary_count) bytes, 16-byte
 *     aligned.
 * Results are bitwise reproducible and do not depend on the grid size. batch must be > 0
 * (the loss of an empty interior set is undefined).
 *
 * Replaces, as one call, the Python training step of
 * /root/reference/benchmarks/train_poisson.py:30-45 and
 * /root/reference/benchmarks/benchmark_training.py:41-60:
 *   - fused_forward_laplacian_cuda (csrc/fused_residual.cu:587-643);
 *   - the loss of src/fused_hoad/training.py:66-88 and its autograd backward;
 *   - fused_forward_laplacian_backward_cuda (csrc/fused_backward.cu:859-934);
 *   - the differentiable pack (src/fused_hoad/parameters.py:77-78);
 *   - torch.optim.Adam.step.
 */
int fhoad_poisson_adam_step(const float* coordinates, const float* source, int64_t batch,
                            const float* boundary, int64_t boundary_count, double boundary_weight,
                            float* parameters, float* exp_avg, float* exp_avg_sq, float* step,
                            float* loss, float* grad_parameters, float* grad_coordinates,
                            void* workspace, size_t workspace_bytes, double lr, double beta1,
                            double beta2, double eps, double weight_decay, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FUSED_HOAD_H_ */
