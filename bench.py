"""Benchmark of the fused forward-Laplacian path on one MI355X.

Metric: residual points/s (u, Laplacian u) at 64K points plus train-step ms at
64K points, FP32, 1 GPU. One "step" is one fused residual evaluation of 65,536 points
(coordinates already in HBM). The training step (forward jet, loss mean((Laplacian u - f)^2)
with f = -2 pi^2 sin(pi x) sin(pi y), adjoint jet, Adam lr 1e-3) is timed the same way at 65,536
points with all of BASELINE config 3's outputs (gradients of every weight and bias and of the
input coordinates): ``train_step_ms`` is the fused step (FusedPoissonAdam: one gradient kernel
that re-runs the forward and seeds itself from the loss, one reduction kernel with the Adam
update), ``train_step_graphed_ms`` the same replayed from a HIP graph, and
``train_step_autograd_ms`` the reference's step through the drop-in API (fused forward +
autograd loss + fused backward + torch.optim.Adam) on a model flattened once with
``flatten_poisson_parameters_`` (``train_step_autograd_unflattened_ms``: on the model as
built), ``train_step_autograd_graphed_ms`` that drop-in step captured whole in a HIP graph
(the reference's "whole step CUDA-graph captured" row), and
``train_step_autograd_graphed_fused_adam_ms`` the same with ``torch.optim.Adam(fused=True)``
(``..._saved_ms``: also with ``backward="saved"``). ``saving_forward_ms`` and
``saved_backward_call_ms`` time the opt-in saved-layer pair (the forward keeps the hidden
layers, 3 KB per point; the backward reads them instead of re-running the forward).
``train_step_no_coordinate_grad_ms`` is the fused step without the coordinate gradient, a
labelled variant only.

``host_us_per_call`` is host time per call at 64 points (no synchronize inside a loop of 2,000
calls, the method of the reference's benchmarks/host_overhead.py): the fused call under no_grad
(the reference quotes 16-20 us, README.md:102) and zero_grad + forward + backward of
``fused_laplacian`` on a flattened model and on the model as built. ``launches_per_step``
counts, with torch.profiler as the reference's benchmarks/count_launches.py does, the host launch
calls and GPU kernels of one drop-in step, one fused step and one graph-replayed fused step at
the training size.

``cpu_baseline`` times the reference's CPU path on the host's cores: the headline residual in
the reference's op structure (one stacked [batch, 4, 64] jet with in-place row fix-ups,
oracle/torch_ref.py forward_laplacian_stacked), the four-matmul restatement beside it, and the
eager nested-autograd training step.

``roofline.traffic`` comes from the committed rocprofv3 summary
profiles/forward_kernel_65536_traffic.json only when that was measured on the kernel source
this run executes (same SHA-256); otherwise it is null and ``traffic_source`` says why.

Timing: the residual first runs untimed for --settle-seconds (0.3 s by default), because the
shader clock needs about 0.1 s of sustained load to reach its steady level and a few warmup
calls alone would time a GPU that is still ramping. Each quantity is then W warmup calls and K
calls run back to back between two synchronizes; `value` and the step times come from the host
clock over those K calls, and each kernel's average duration (the
roofline's `avg_launch_ms`) from one HIP event pair on the launch stream around the same calls.
A separate pass with an event pair per call gives the median and p90 in the log only (per-call
event packets add their own time to each call).

Correctness is checked before any timing: the fused forward against the package's PyTorch
forward Laplacian (atol 1e-5 / rtol 1e-4) and the fused backward against the PyTorch
recompute backward (1e-4 of each gradient block's scale); a mismatch aborts.

Prints human-readable lines to stderr and ONE JSON line to stdout.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "expanded-gpu-optimization_amd"))

METRIC = "residual points/sec (u,Δu) at 64K + train-step ms at 64K, FP32, 1 GPU"
PEAK_FP32_MATRIX_TFLOPS = 157.3  # MI355X dense FP32 MFMA (256 CUs x 256 FLOP/clk x 2.4 GHz)
FLOP_PER_POINT_FORWARD = 3 * 64 * 64 * 4 * 2  # hidden-layer contractions: 98,304
FLOP_PER_POINT_BACKWARD = 2 * FLOP_PER_POINT_FORWARD  # dW + hbar (recompute not counted)
REFERENCE_A5000 = {"residual_points_per_s_64k": 121.9e6, "train_step_ms_64k": 3.334,
                   "hardware": "RTX A5000", "source": "reference results/2026-11-06-RTX-A5000-8454035"}
TRAFFIC_FILE = ROOT / "profiles" / "forward_kernel_65536_traffic.json"
KERNEL_SOURCE = ROOT / "expanded-gpu-optimization_amd" / "csrc" / "fused_hoad_kernels.hip"
CPU_RESIDUAL_CALLS = 100     # CPU baseline sample sizes (see _cpu_baseline)
CPU_RESIDUAL_1K_CALLS = 200
CPU_STEP_CALLS = 40


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def _parse() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--points", type=int, default=65536)
    parser.add_argument("--train-points", type=int, default=65536)
    parser.add_argument("--settle-seconds", type=float, default=0.3,
                        help="untimed residual calls before any timing, for the clock to settle")
    parser.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--kernels-only", action="store_true",
                        help="after the correctness check, time only the fused forward and backward "
                             "calls (for counter collection); prints no JSON line")
    parser.add_argument("--no-host-overheads", action="store_true",
                        help="skip the host-time and launch-count passes (profiled runs: under "
                             "rocprofv3 --pmc the 2,000-call host-time loop's deep queue of tiny "
                             "dispatches was aborted with a malformed AQL packet)")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="also run a plain device copy of this many MiB (rocprof counter scale)")
    args = parser.parse_args()
    if args.steps < 1 or args.warmup < 0 or args.points < 1 or args.train_points < 1 or args.settle_seconds < 0:
        parser.error("steps and points must be positive, warmup and settle-seconds non-negative")
    return args


def _gpu_clock_mhz() -> float | None:
    """Active shader-clock level from the amdgpu sysfs table (the line marked '*'), best
    effort and without starting any process."""
    for table in sorted(Path("/sys/class/drm").glob("card*/device/pp_dpm_sclk")):
        try:
            for line in table.read_text().splitlines():
                if line.rstrip().endswith("*"):
                    return float(line.split(":", 1)[1].strip().lower().split("mhz")[0])
        except (OSError, ValueError, IndexError):
            continue
    return None


def _settle(fn, seconds: float, torch) -> None:
    """Run `fn` untimed for about `seconds` (in bursts of 20 calls)."""
    deadline = time.perf_counter() + seconds
    while time.perf_counter() < deadline:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


def _timed(fn, iterations: int, torch):
    """Run fn `iterations` times back to back, bracketed by synchronize, with one HIP event
    pair on the current stream (the stream the kernels run on) around the whole region.
    Returns (wall_ms, gpu_ms) totals. Nothing is recorded between calls, so the calls run as a
    caller would run them."""
    stream = torch.cuda.current_stream()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start = time.perf_counter()
    begin.record(stream)
    for _ in range(iterations):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return (time.perf_counter() - start) * 1e3, begin.elapsed_time(end)


def _per_call_events(fn, iterations: int, torch) -> list[float]:
    """Per-call HIP event pairs (ms), for the median and p90 in the log; the event packets
    between calls add their own time, so these are not used for `value`."""
    stream = torch.cuda.current_stream()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iterations)]
    torch.cuda.synchronize()
    for begin, end in pairs:
        begin.record(stream)
        fn()
        end.record(stream)
    torch.cuda.synchronize()
    return [b.elapsed_time(e) for b, e in pairs]


def _p90(samples: list[float]) -> float:
    ordered = sorted(samples)
    return ordered[min(len(ordered) - 1, int(0.9 * len(ordered)))]


def _kernel_source_sha256() -> str:
    return hashlib.sha256(KERNEL_SOURCE.read_bytes()).hexdigest()


def _measured_traffic(points: int):
    """HBM bytes per forward launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary, used only when it was measured on this workload AND on the kernel source this
    run executes (its SHA-256 is recorded in the file); otherwise None, with the reason."""
    if not TRAFFIC_FILE.exists():
        return None, "no committed measurement"
    measured = json.loads(TRAFFIC_FILE.read_text())
    where = str(TRAFFIC_FILE.relative_to(ROOT))
    if measured.get("points") != points:
        return None, f"{where} holds {measured.get('points')} points, not {points}"
    current = _kernel_source_sha256()
    if measured.get("kernel_source_sha256") != current:
        return None, (f"stale: {where} was measured on kernel source "
                      f"{str(measured.get('kernel_source_sha256'))[:12]}, this run's is {current[:12]}")
    return measured.get("hbm_bytes_per_launch"), {
        "file": where, "kernel_source_sha256": current, "commands": measured.get("commands"),
    }


def _host_us(fn, calls: int, torch, repeats: int = 5) -> float:
    """Host time per call in us: `calls` calls with no synchronize inside the loop, divided by
    `calls` (/root/reference/benchmarks/host_overhead.py:27-35); the median of `repeats` such
    loops."""
    samples = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        tick = time.perf_counter()
        for _ in range(calls):
            fn()
        samples.append((time.perf_counter() - tick) * 1e6 / calls)
        torch.cuda.synchronize()
    return round(statistics.median(samples), 2)


def _host_overheads(torch, device, get_backend, fused_laplacian, flatten) -> dict:
    """Host time per call at 64 points, where the kernels are short and the host dominates:
    the reference's fused call (the fused_cuda backend under no_grad, README.md:102 quotes
    16-20 us on its hosts), and zero_grad + forward + backward of fused_laplacian with a small
    loss on a flattened model and on the model as built."""
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp

    calls = 2000
    gen = torch.Generator().manual_seed(0)
    x = (torch.rand(64, 2, generator=gen) * 2 - 1).to(device)
    torch.manual_seed(0)
    frozen = build_mlp(DEFAULT_POISSON_MLP).to(device).requires_grad_(False)
    run = get_backend("fused_cuda")
    with torch.no_grad():
        for _ in range(50):
            run(frozen, x)
        forward_us = _host_us(lambda: run(frozen, x), calls, torch)
    result = {"batch": 64, "calls": calls, "forward_no_grad": forward_us}
    for label, flat in (("forward_backward_flattened", True), ("forward_backward_as_built", False)):
        torch.manual_seed(0)
        model = build_mlp(DEFAULT_POISSON_MLP).to(device)
        if flat:
            flatten(model)

        def step():
            model.zero_grad(set_to_none=True)
            _, lap = fused_laplacian(model, x)
            lap.pow(2).mean().backward()

        for _ in range(50):
            step()
        result[label] = _host_us(step, calls, torch)
    return result


_LAUNCH_MARKERS = ("LaunchKernel", "GraphLaunch", "LaunchCooperativeKernel")


def _launch_counts(torch, fn) -> dict:
    """Host launch calls and GPU kernels of one call of `fn`, counted with torch.profiler as
    the reference does (/root/reference/benchmarks/count_launches.py:15-38): runtime launch
    API events on the CPU side, kernel events on the GPU side."""
    from torch.profiler import ProfilerActivity, profile

    try:
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        events = prof.events()
        launch_names = sorted({e.name for e in events if any(k in e.name for k in _LAUNCH_MARKERS)})
        launches = sum(1 for e in events if any(k in e.name for k in _LAUNCH_MARKERS))
        device = [e.name for e in events if e.device_type == torch.autograd.DeviceType.CUDA
                  and "#" not in e.name]  # user annotations (Optimizer.step#...) are not GPU work
        copies = [n for n in device if n.startswith(("Memcpy", "Memset"))]
        kernels = [n for n in device if not n.startswith(("Memcpy", "Memset"))]
        return {"host_launches": launches, "gpu_kernels": len(kernels), "gpu_copies": len(copies),
                "launch_calls": launch_names,
                "kernels": sorted({n.split("(")[0][-80:] for n in kernels})}
    except Exception as err:  # the profiler is a measurement aid: report, do not abort the bench
        return {"host_launches": None, "gpu_kernels": None, "error": f"{type(err).__name__}: {err}"}


def _scaled_error(actual, expected) -> float:
    return float((actual - expected).abs().max() / expected.abs().max().clamp_min(1e-30))


def main() -> None:
    args = _parse()
    if args.gpus != 1:
        log(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the path is data-parallel "
            "over points and its multi-GPU design is described, not run. Use --gpus 1.")
        sys.exit(2)

    import torch

    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp, forward_laplacian, get_backend, manufactured_source
    from fused_hoad._extension import (
        fused_forward_laplacian,
        fused_forward_laplacian_backward,
        load_extension,
    )
    from fused_hoad.backends.fused import _recompute_backward, fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_, pack_poisson_parameters
    from fused_hoad.training import FusedPoissonAdam, cuda_graph_step

    load_extension()  # fail loudly if the HIP extension is missing
    if not torch.cuda.is_available():
        raise SystemExit("no GPU visible")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    props = torch.cuda.get_device_properties(device)
    log(f"device: {props.name} ({getattr(props, 'gcnArchName', '?')}), CUs={props.multi_processor_count}, "
        f"torch {torch.__version__}, hip {torch.version.hip}")

    # ---- inputs: seeded model, coordinates U[-1,1]^2 from a seeded CPU generator ----
    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP).to(device)
    params = pack_poisson_parameters(model)
    gen = torch.Generator().manual_seed(0)
    x = (torch.rand(args.points, 2, generator=gen) * 2 - 1).to(device)
    x_train = (torch.rand(args.train_points, 2, generator=gen) * 2 - 1).to(device)

    # ---- correctness before timing ----
    with torch.no_grad():
        u, lap = fused_forward_laplacian(x, params)
        eu, el = forward_laplacian(model, x)
    torch.testing.assert_close(u, eu, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(lap, el, atol=1e-5, rtol=1e-4)
    gu = torch.zeros(args.train_points, 1, device=device)
    gl = torch.randn(args.train_points, 1, device=device, generator=torch.Generator(device=device).manual_seed(1))
    gp, gx = fused_forward_laplacian_backward(x_train, params, gu, gl)
    ex, ep = _recompute_backward(x_train, params, gu, gl, True, True)
    bwd_err = max(_scaled_error(gp, ep), _scaled_error(gx, ex))
    if bwd_err > 1e-4:
        raise SystemExit(f"fused backward disagrees with the recompute backward: {bwd_err:.3e}")
    log(f"check: forward within atol 1e-5/rtol 1e-4, backward max scaled error {bwd_err:.2e}")

    # ---- residual: K fused forward calls ----
    def residual_step():
        fused_forward_laplacian(x, params)

    # Measured at 64K points: 59 us per call after 10 warmup calls, 53 us after 2,000 (0.1 s).
    _settle(residual_step, args.settle_seconds, torch)
    for _ in range(args.warmup):
        residual_step()
    total_ms, gpu_ms = _timed(residual_step, args.steps, torch)
    ms_per_step = total_ms / args.steps
    fwd_kernel_ms = gpu_ms / args.steps
    points_per_s = args.points / (ms_per_step / 1e3)
    per_call = _per_call_events(residual_step, args.steps, torch)
    log(f"residual {args.points} pts: {ms_per_step * 1e3:.1f} us/step wall, {fwd_kernel_ms * 1e3:.1f} us/call "
        f"(GPU events over the {args.steps} calls), {points_per_s / 1e6:.1f} M points/s; per-call events: "
        f"median {statistics.median(per_call) * 1e3:.1f} us, p90 {_p90(per_call) * 1e3:.1f} us")

    # ---- backward call alone (backward kernel + fixed-order reduction) ----
    def backward_step():
        fused_forward_laplacian_backward(x_train, params, gu, gl)

    for _ in range(args.warmup):
        backward_step()
    _, bwd_gpu_ms = _timed(backward_step, args.steps, torch)
    bwd_ms = bwd_gpu_ms / args.steps

    if args.kernels_only:
        log(f"backward call {args.train_points} pts: {bwd_ms * 1e3:.1f} us (GPU events over the calls)")
        return

    # ---- the saved-layer pair (opt-in "saved" mode): a forward that keeps the hidden layers
    # (3 KB per point) and a backward that reads them instead of re-running the forward. Checked
    # bitwise against the pair above first; timed the same way, each call alone.
    ext = load_extension()
    gu_flat, gl_flat = gu.reshape(-1).contiguous(), gl.reshape(-1).contiguous()
    ref_u, ref_lap = fused_forward_laplacian(x_train, params)
    saved_u, saved_lap, saved_layers = ext._forward_saving(x_train, params, 2)
    ref_gp, ref_gx = ext._backward(x_train, params, gu_flat, gl_flat, True, 6)
    saved_gp, saved_gx = ext._backward(x_train, params, gu_flat, gl_flat, True, 6, saved_layers)
    if not (torch.equal(saved_u, ref_u) and torch.equal(saved_lap, ref_lap)
            and torch.equal(saved_gp, ref_gp) and torch.equal(saved_gx, ref_gx)):
        raise SystemExit("the saved-layer pair differs from the forward and backward calls")

    def forward_train_step():
        fused_forward_laplacian(x_train, params)

    def saving_forward_step():
        ext._forward_saving(x_train, params, 2)

    def saved_backward_step():
        ext._backward(x_train, params, gu_flat, gl_flat, True, 6, saved_layers)

    pair_ms = {}
    for name, fn in (("forward", forward_train_step), ("saving_forward", saving_forward_step),
                     ("saved_backward", saved_backward_step)):
        for _ in range(args.warmup):
            fn()
        _, gpu = _timed(fn, args.steps, torch)
        pair_ms[name] = gpu / args.steps
    del saved_layers
    log(f"saved-layer pair {args.train_points} pts: saving forward {pair_ms['saving_forward'] * 1e3:.1f} us "
        f"(forward {pair_ms['forward'] * 1e3:.1f} us), saved-layer backward {pair_ms['saved_backward'] * 1e3:.1f} us "
        f"(backward {bwd_ms * 1e3:.1f} us); forward + backward {(pair_ms['forward'] + bwd_ms) * 1e3:.1f} us, "
        f"saved pair {(pair_ms['saving_forward'] + pair_ms['saved_backward']) * 1e3:.1f} us; bitwise the same results")

    # ---- training step (a): the reference's step through the drop-in API ----
    # fused forward (the C++ autograd Function behind fused_laplacian) + mean((Lap u - f)^2) +
    # fused backward + torch Adam (/root/reference/benchmarks/benchmark_training.py:41-60).
    # train_step_autograd_ms runs it on a model flattened once with flatten_poisson_parameters_
    # (its parameters become views of the packed buffer, so fused_laplacian packs nothing per
    # step); train_step_autograd_unflattened_ms on the model as built (one pack copy per step,
    # inside the Function).
    source = manufactured_source(x_train)

    def autograd_timing(flatten: bool) -> float:
        torch.manual_seed(0)
        step_model = build_mlp(DEFAULT_POISSON_MLP).to(device)
        if flatten:
            flatten_poisson_parameters_(step_model)
        optimizer = torch.optim.Adam(step_model.parameters(), lr=1e-3)

        def autograd_step():
            optimizer.zero_grad(set_to_none=True)
            _, lap_t = fused_laplacian(step_model, x_train)
            (lap_t - source).pow(2).mean().backward()
            optimizer.step()

        for _ in range(args.warmup):
            autograd_step()
        total_ms, _ = _timed(autograd_step, args.steps, torch)
        return total_ms / args.steps

    autograd_ms = autograd_timing(True)
    autograd_unflattened_ms = autograd_timing(False)
    log(f"train step (autograd drop-in) {args.train_points} pts: {autograd_ms:.3f} ms wall/step "
        f"(flattened model), {autograd_unflattened_ms:.3f} ms (unflattened)")

    # The same drop-in step captured whole in a HIP graph (cuda_graph_step: forward, autograd
    # loss and backward, Adam with capturable=True), the form of the reference's "whole step
    # CUDA-graph captured" row. Before timing, every replay of a short run is checked against
    # the same steps run eagerly from the same weights (the loss each step, rtol 1e-4, and the
    # weights after); a graph that replays wrongly is not timed (the field is null and
    # train_step_autograd_graphed_note says why).
    def autograd_graph_timing(fused_adam: bool, mode: str = "cuda"):
        def make():
            torch.manual_seed(0)
            model = build_mlp(DEFAULT_POISSON_MLP).to(device)
            flatten_poisson_parameters_(model)
            return model

        def loss_of(model):
            def loss_fn():
                _, lap_t = fused_laplacian(model, x_train, backward=mode)
                return (lap_t - source).pow(2).mean()
            return loss_fn

        graph_model, eager_model = make(), make()
        if fused_adam:
            graph_opt = torch.optim.Adam(graph_model.parameters(), lr=1e-3, fused=True, capturable=True)
            eager_opt = torch.optim.Adam(eager_model.parameters(), lr=1e-3, fused=True)
        else:
            graph_opt = torch.optim.Adam(graph_model.parameters(), lr=1e-3, capturable=True)
            eager_opt = torch.optim.Adam(eager_model.parameters(), lr=1e-3)
        replay = cuda_graph_step(loss_of(graph_model), graph_opt, warmup=3)
        eager_loss = loss_of(eager_model)
        for k in range(3 + 10):
            eager_opt.zero_grad(set_to_none=True)
            loss = eager_loss()
            loss.backward()
            eager_opt.step()
            if k >= 3:
                got, want = replay().item(), loss.item()
                if abs(got - want) > 1e-4 * abs(want):
                    return None, f"replay {k - 3} loss {got} differs from the eager step's {want}"
        for a, b in zip(graph_model.parameters(), eager_model.parameters()):
            if not torch.allclose(a, b, rtol=1e-4, atol=1e-6):
                return None, "weights after 10 replays differ from those after 10 eager steps"
        for _ in range(args.warmup):
            replay()
        total_ms, _ = _timed(replay, args.steps, torch)
        return total_ms / args.steps, "10 replays checked against eager steps (loss rtol 1e-4, weights)"

    def checked_graph_timing(fused_adam: bool, mode: str = "cuda"):
        try:
            return autograd_graph_timing(fused_adam, mode)
        except RuntimeError as err:  # a capture this torch build refuses: reported, not fatal
            return None, f"capture failed: {err}"

    autograd_graph_ms, autograd_graph_note = checked_graph_timing(False)
    # labelled variant: the same with torch.optim.Adam(fused=True) (one optimizer kernel)
    autograd_graph_fused_ms, autograd_graph_fused_note = checked_graph_timing(True)
    # labelled variant: the same with backward="saved" (the forward keeps 3 KB per point)
    autograd_graph_saved_ms, autograd_graph_saved_note = checked_graph_timing(True, "saved")
    for label, ms, note in (("foreach Adam", autograd_graph_ms, autograd_graph_note),
                            ("Adam(fused=True)", autograd_graph_fused_ms, autograd_graph_fused_note),
                            ("Adam(fused=True), backward='saved'", autograd_graph_saved_ms,
                             autograd_graph_saved_note)):
        if ms is None:
            log(f"train step (autograd drop-in, whole step in a HIP graph, {label}): not timed, {note}")
        else:
            log(f"train step (autograd drop-in, whole step in a HIP graph, {label}) {args.train_points} pts: "
                f"{ms:.3f} ms wall/step (flattened model; {note})")

    # ---- training step (b): the fused step, FusedPoissonAdam (2 kernels) ----
    # All of config 3's outputs: the gradients of every weight and bias and of the input
    # coordinates (they require grad, so each step writes trainer.grad_coordinates, as the
    # reference's backward always writes grad_coordinates, csrc/fused_backward.cu:830-831).
    torch.manual_seed(0)
    fused_model = build_mlp(DEFAULT_POISSON_MLP).to(device)
    x_train_grad = x_train.detach().clone().requires_grad_(True)
    trainer = FusedPoissonAdam(fused_model, x_train_grad, source, lr=1e-3)
    # check the first step before timing: loss against the fused forward's, parameter and
    # coordinate gradients against the recompute backward seeded with grad_lap = 2 (lap - f) / B
    with torch.no_grad():
        _, lap0 = fused_forward_laplacian(x_train, trainer.parameters)
    resid0 = lap0 - source
    want_loss = resid0.double().pow(2).mean().item()
    want_grad_x, want_grad = _recompute_backward(x_train, trainer.parameters.clone(), torch.zeros_like(lap0),
                                                 2.0 * resid0 / args.train_points, True, True)
    got_loss = trainer.step().item()
    step_err = max(_scaled_error(trainer.grad, want_grad),
                   _scaled_error(trainer.grad_coordinates, want_grad_x))
    if abs(got_loss - want_loss) > 1e-5 * abs(want_loss) or step_err > 1e-4:
        raise SystemExit(f"fused step disagrees: loss {got_loss} vs {want_loss}, gradient {step_err:.3e}")
    log(f"check: fused step loss rel error {abs(got_loss - want_loss) / want_loss:.2e}, "
        f"parameter and coordinate gradients max scaled error {step_err:.2e}")
    for _ in range(args.warmup):
        trainer.step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(device)
    baseline_bytes = torch.cuda.memory_allocated(device)
    train_total_ms, train_gpu_ms = _timed(trainer.step, args.steps, torch)
    train_ms = train_total_ms / args.steps
    peak_mib = (torch.cuda.max_memory_allocated(device) - baseline_bytes) / 2**20
    train_calls = _per_call_events(trainer.step, args.steps, torch)
    log(f"train step (fused, with coordinate gradients) {args.train_points} pts: {train_ms:.3f} ms wall/step, "
        f"{train_gpu_ms / args.steps:.3f} ms GPU/step; per-call events median {statistics.median(train_calls):.3f} ms, "
        f"p90 {_p90(train_calls):.3f} ms; backward call {bwd_ms * 1e3:.1f} us; peak {peak_mib:.1f} MiB above baseline")

    # labelled variant: the same step on coordinates that do not require grad (no
    # grad_coordinates store), for comparison with earlier records only
    torch.manual_seed(0)
    plain_trainer = FusedPoissonAdam(build_mlp(DEFAULT_POISSON_MLP).to(device), x_train, source, lr=1e-3)
    for _ in range(args.warmup + 1):
        plain_trainer.step()
    plain_total_ms, _ = _timed(plain_trainer.step, args.steps, torch)
    plain_ms = plain_total_ms / args.steps
    log(f"train step (fused, no coordinate gradients) {args.train_points} pts: {plain_ms:.3f} ms wall/step")
    del plain_trainer

    # ---- training step (c): the fused step replayed from a HIP graph ----
    replay = trainer.graphed(warmup=1)
    for _ in range(args.warmup):
        replay()
    graph_total_ms, _ = _timed(replay, args.steps, torch)
    graph_ms = graph_total_ms / args.steps
    log(f"train step (fused, HIP graph) {args.train_points} pts: {graph_ms:.3f} ms wall/step")

    # ---- host time per call and launches per step (the reference's host_overhead.py and
    # count_launches.py methods) ----
    host_us, launches = None, None
    if not args.no_host_overheads:
        host_us = _host_overheads(torch, device, get_backend, fused_laplacian, flatten_poisson_parameters_)
        log("host time per call at 64 points (us, median of 5 x 2,000 calls, no sync inside): "
            + ", ".join(f"{k} {v}" for k, v in host_us.items() if isinstance(v, float)))
        torch.manual_seed(0)
        dropin_model = build_mlp(DEFAULT_POISSON_MLP).to(device)
        flatten_poisson_parameters_(dropin_model)
        dropin_opt = torch.optim.Adam(dropin_model.parameters(), lr=1e-3)

        def dropin_step():
            dropin_opt.zero_grad(set_to_none=True)
            _, lap_t = fused_laplacian(dropin_model, x_train)
            (lap_t - source).pow(2).mean().backward()
            dropin_opt.step()

        launches = {
            "drop_in_step": _launch_counts(torch, dropin_step),
            "fused_step": _launch_counts(torch, trainer.step),
            "fused_step_graph": _launch_counts(torch, replay),
        }
        log("launches per step (host launch calls / GPU kernels, torch.profiler): "
            + ", ".join(f"{k} {v.get('host_launches')}/{v.get('gpu_kernels')}" for k, v in launches.items()))

    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * 2**20 // 4
        src = torch.ones(n, device=device)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration: copied {args.calibrate_copy_mib} MiB 5 times")

    clock = _gpu_clock_mhz()
    fwd_tflops = FLOP_PER_POINT_FORWARD * args.points / (fwd_kernel_ms / 1e3) / 1e12
    bwd_tflops = FLOP_PER_POINT_BACKWARD * args.train_points / (bwd_ms / 1e3) / 1e12
    traffic, traffic_source = _measured_traffic(args.points)
    roofline = {
        "bound": "mfma",
        "achieved": round(fwd_tflops, 3),
        "peak": PEAK_FP32_MATRIX_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(fwd_tflops / PEAK_FP32_MATRIX_TFLOPS, 4),
        "traffic": traffic,
        "traffic_source": traffic_source,
        "kernel": "forward_kernel",
        "flop_per_launch": FLOP_PER_POINT_FORWARD * args.points,
        "avg_launch_ms": round(fwd_kernel_ms, 5),
        "avg_launch_ms_from": "HIP events on the launch stream around the timed calls, divided by the call count",
    }
    roofline_backward = {
        "bound": "mfma",
        "achieved": round(bwd_tflops, 3),
        "peak": PEAK_FP32_MATRIX_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(bwd_tflops / PEAK_FP32_MATRIX_TFLOPS, 4),
        "kernel": "backward_kernel + reduce_partials_kernel (one backward call)",
        "flop_per_launch": FLOP_PER_POINT_BACKWARD * args.train_points,
        "avg_launch_ms": round(bwd_ms, 5),
    }
    step_flop = (FLOP_PER_POINT_FORWARD + FLOP_PER_POINT_BACKWARD) * args.train_points
    train_tflops = step_flop / (train_ms / 1e3) / 1e12
    roofline_train_step = {
        "bound": "mfma",
        "achieved": round(train_tflops, 3),
        "peak": PEAK_FP32_MATRIX_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(train_tflops / PEAK_FP32_MATRIX_TFLOPS, 4),
        "kernel": "fused step: backward_kernel<loss> + reduce_adam_kernel, wall time per step",
        "flop_per_step": step_flop,
    }

    cpu_baseline = None
    if not args.no_cpu_baseline:
        cpu_baseline = _cpu_baseline(torch)

    record = {
        "metric": METRIC,
        "value": round(points_per_s, 1),
        "unit": "points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_seconds": args.settle_seconds,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (coordinates U[-1,1]^2 from a seeded CPU generator; torch.manual_seed(0) default nn.Linear init)",
        "config": {
            "workload": "fused residual (u, Laplacian u) of the 2->64x4->1 tanh MLP at 65,536 points; "
                        "train step = forward jet + mean((Lap u - f)^2) + adjoint jet + Adam(lr 1e-3) at 65,536 points "
                        "(train_step_ms: the fused step, FusedPoissonAdam; train_step_autograd_ms: the same step "
                        "through fused_laplacian + autograd + torch.optim.Adam)",
            "points": args.points,
            "train_points": args.train_points,
        },
        "train_step_ms": round(train_ms, 5),
        "train_step_outputs": "loss, gradients of all 12,737 parameters and of the 65,536 x 2 input coordinates, Adam update",
        "train_step_no_coordinate_grad_ms": round(plain_ms, 5),
        "train_step_tflops": round(train_tflops, 3),
        "train_step_peak_mib": round(peak_mib, 2),
        "train_step_graphed_ms": round(graph_ms, 5),
        "train_step_autograd_ms": round(autograd_ms, 5),
        "train_step_autograd_unflattened_ms": round(autograd_unflattened_ms, 5),
        "train_step_autograd_graphed_ms": None if autograd_graph_ms is None else round(autograd_graph_ms, 5),
        "train_step_autograd_graphed_note": autograd_graph_note,
        "train_step_autograd_graphed_fused_adam_ms": (None if autograd_graph_fused_ms is None
                                                      else round(autograd_graph_fused_ms, 5)),
        "train_step_autograd_graphed_fused_adam_saved_ms": (None if autograd_graph_saved_ms is None
                                                            else round(autograd_graph_saved_ms, 5)),
        "saving_forward_ms": round(pair_ms["saving_forward"], 5),
        "saved_backward_call_ms": round(pair_ms["saved_backward"], 5),
        "backward_call_ms": round(bwd_ms, 5),
        "gpu_clock_mhz": clock,
        "roofline": roofline,
        "roofline_backward": roofline_backward,
        "roofline_train_step": roofline_train_step,
        "host_us_per_call": host_us,
        "launches_per_step": launches,
        "cpu_baseline": cpu_baseline,
        "reference_published": REFERENCE_A5000,
    }
    print(json.dumps(record), flush=True)


def _cpu_description() -> dict:
    """The host CPU as /proc/cpuinfo describes it (model name, vendor, family/model/stepping,
    MHz), plus the logical CPU count."""
    fields = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" not in line:
                if fields:
                    break  # the first processor's block is enough
                continue
            key, value = (part.strip() for part in line.split(":", 1))
            if key in ("model name", "vendor_id", "cpu family", "model", "stepping", "cpu MHz") and key not in fields:
                fields[key] = value
    except OSError:
        pass
    model = fields.get("model name", "?")
    detail = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping", "cpu MHz")
                       if k in fields)
    return {"cpu_model": f"{model} ({detail})" if detail else model, "os_cpu_count": os.cpu_count()}


def _cpu_baseline(torch) -> dict:
    """The reference's CPU path (oracle/torch_ref.py, a restatement of its PyTorch forward
    Laplacian and eager-autograd training step) on this host's cores, on a bounded sample. The
    headline residual is the reference's op structure (forward_laplacian_stacked: one stacked
    [batch, 4, 64] jet with in-place row fix-ups); the four-matmul restatement is timed beside it."""
    sys.path.insert(0, str(ROOT))
    from oracle import torch_ref

    threads = torch.get_num_threads()
    model = torch_ref.reference_model(0)
    flat = torch_ref.pack(model)
    gen = torch.Generator().manual_seed(0)
    x = torch.rand(65536, 2, generator=gen) * 2 - 1
    x1k = x[:1024].contiguous()

    def median_ms(fn, warmup, iterations):
        for _ in range(warmup):
            fn()
        samples = []
        for _ in range(iterations):
            tick = time.perf_counter()
            fn()
            samples.append((time.perf_counter() - tick) * 1e3)
        return statistics.median(samples)

    # About 15 s of CPU work in all on a 16-thread host (each 64K residual form about 4 s, the
    # eager step about 5 s), so that the medians are stable and the bench still ends within
    # minutes.
    with torch.no_grad():
        stacked64k_ms = median_ms(lambda: torch_ref.forward_laplacian_stacked(flat, x), 2, CPU_RESIDUAL_CALLS)
        stacked1k_ms = median_ms(lambda: torch_ref.forward_laplacian_stacked(flat, x1k), 5, CPU_RESIDUAL_1K_CALLS)
        split64k_ms = median_ms(lambda: torch_ref.forward_laplacian(flat, x), 2, CPU_RESIDUAL_CALLS)
    optimizer = torch.optim.Adam(model.parameters(), lr=1e-3)
    source = torch_ref.poisson_source(x)
    step_ms = median_ms(lambda: torch_ref.eager_train_step(model, x, source, optimizer), 2, CPU_STEP_CALLS)
    cpu = _cpu_description()
    log(f"cpu baseline ({threads} threads, os.cpu_count()={cpu['os_cpu_count']}, {cpu['cpu_model']}): "
        f"forward Laplacian (stacked jet, the reference's ops) 64K {stacked64k_ms:.1f} ms, 1K {stacked1k_ms:.2f} ms; "
        f"four-matmul restatement 64K {split64k_ms:.1f} ms; eager step 64K {step_ms:.1f} ms")
    return {
        "value": round(65536 / (stacked64k_ms / 1e3), 1),
        "unit": "points/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle/torch_ref.py forward_laplacian_stacked (the reference's op structure: one stacked "
                  f"[batch, 4, 64] jet, in-place row fix-ups) (u, Lap u) at 65,536 points, median of "
                  f"{CPU_RESIDUAL_CALLS} calls after 2 warmup ({stacked64k_ms:.1f} ms/call); 1,024 points: "
                  f"{stacked1k_ms:.2f} ms/call (median of {CPU_RESIDUAL_1K_CALLS}); the four-matmul restatement "
                  f"(forward_laplacian) at 65,536 points: {split64k_ms:.1f} ms/call; eager nested-autograd + Adam "
                  f"train step at 65,536 points: {step_ms:.1f} ms/step (median of {CPU_STEP_CALLS})",
        "residual_64k_ms": round(stacked64k_ms, 3),
        "residual_1k_ms": round(stacked1k_ms, 4),
        "residual_64k_four_matmul_ms": round(split64k_ms, 3),
        "train_step_ms": round(step_ms, 3),
        "os_cpu_count": cpu["os_cpu_count"],
        "cpu_model": cpu["cpu_model"],
    }


if __name__ == "__main__":
    main()
