"""Per-phase clock of the backward kernel, from the measurement build of the library.

``python -m fused_hoad._build --phase-clock`` (any host with hipcc) compiles
``libfused_hoad_hip_phase_clock.so``: the same kernels with ``-DFHOAD_PHASE_CLOCK``, where each
wave of the backward kernel adds the shader-clock cycles it spends in each phase of its tiles
to a device table. This script (on a GPU) runs one workload through that library's C ABI a
number of times, reads the table after each call and prints, as Markdown, the median over
calls of each phase's cycles per wave and per tile, with the wall-clock span of the kernel.

Workloads:

* ``step``: ``fhoad_poisson_adam_step`` with ``--batch`` interior and ``--boundary`` boundary
  points (the PINN training step; its gradient kernel is the backward kernel with the loss);
* ``backward``: ``fhoad_forward_laplacian_backward`` at ``--batch`` points.

The clock reads wait for each wave's outstanding LDS reads at the phase boundaries, so the
measured kernel is somewhat slower than the library's; the table gives the span of both
(``--compare`` times the library build's kernel with HIP events on the same inputs).
Nothing in the package imports this module.
"""

from __future__ import annotations

import argparse
import ctypes
import statistics
import sys
from pathlib import Path

import torch

PACKAGE_DIR = Path(__file__).resolve().parent
CLOCK_LIBRARY = PACKAGE_DIR / "libfused_hoad_hip_phase_clock.so"
LIBRARY = PACKAGE_DIR / "libfused_hoad_hip.so"

# Field order of ClockField in csrc/fused_hoad_kernels.hip.
PHASES = [
    ("stage", "parameter staging (kernel start)"),
    ("forward", "layer 0, hidden layers 1-2 forward (re-run)"),
    ("layer3", "hidden layer 3 forward, loss and output seed, zbar3 staged"),
    ("dw3", "dW3 (three staged passes)"),
    ("adjoint3", "W3^T zbar3"),
    ("dw2", "dW2"),
    ("adjoint2", "W2^T zbar2, layer 0 rebuilt"),
    ("dw1", "dW1"),
    ("layer0", "W1^T zbar1, layer 0 adjoint, coordinate gradients"),
    ("rest", "16-point split tiles past the last whole round"),
    ("boundary", "boundary tiles"),
    ("partials", "partial row of the slot"),
]
TILES, BOUNDARY_TILES, WALL_START, WALL_END = 12, 13, 14, 15
FIELDS = 16
WALL_MHZ = 100.0  # s_memrealtime


def _load(path: Path) -> ctypes.CDLL:
    if not path.exists():
        raise SystemExit(f"{path.name} is not built: run python -m fused_hoad._build --phase-clock")
    lib = ctypes.CDLL(str(path))
    lib.fhoad_last_error.restype = ctypes.c_char_p
    lib.fhoad_backward_workspace_size.restype = ctypes.c_size_t
    lib.fhoad_backward_workspace_size.argtypes = [ctypes.c_int64]
    lib.fhoad_poisson_adam_step_workspace_size.restype = ctypes.c_size_t
    lib.fhoad_poisson_adam_step_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int64]
    p = ctypes.c_void_p
    lib.fhoad_forward_laplacian_backward.argtypes = [
        p, p, p, p, p, p, p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int, p]
    lib.fhoad_poisson_adam_step.argtypes = [
        p, p, ctypes.c_int64, p, ctypes.c_int64, ctypes.c_double, p, p, p, p, p, p, p, p,
        ctypes.c_size_t, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double,
        ctypes.c_double, p]
    return lib


def _check(lib: ctypes.CDLL, status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed ({status}): {lib.fhoad_last_error().decode()}")


def _workload(args: argparse.Namespace):
    """Inputs on cuda:0 and a function that runs one call of `lib` on them."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    dev = torch.device("cuda", 0)
    params = (torch.randn(12737, generator=gen) * 0.2).to(dev)
    coords = (torch.rand(args.batch, 2, generator=gen) * 2 - 1).to(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    if args.workload == "backward":
        grad_out = torch.randn(args.batch, generator=gen).to(dev)
        grad_lap = torch.randn(args.batch, generator=gen).to(dev)
        grad_params = torch.empty(12737, device=dev)
        grad_coords = torch.empty(args.batch, 2, device=dev)

        def run(lib: ctypes.CDLL) -> None:
            size = lib.fhoad_backward_workspace_size(args.batch)
            ws = torch.empty(size // 4 + 4, device=dev)
            _check(lib, lib.fhoad_forward_laplacian_backward(
                ptr(coords), ptr(params), ptr(grad_out), ptr(grad_lap), ptr(grad_params),
                ptr(grad_coords), ptr(ws), size, args.batch, 1, stream), "backward")

        return run
    source = torch.randn(args.batch, generator=gen).to(dev)
    boundary = (torch.rand(max(args.boundary, 1), 2, generator=gen) * 2 - 1).to(dev)
    exp_avg = torch.zeros(12737, device=dev)
    exp_avg_sq = torch.zeros(12737, device=dev)
    step = torch.zeros(1, device=dev)
    loss = torch.empty(1, device=dev)

    def run(lib: ctypes.CDLL) -> None:
        size = lib.fhoad_poisson_adam_step_workspace_size(args.batch, args.boundary)
        ws = torch.empty(size // 4 + 4, device=dev)
        _check(lib, lib.fhoad_poisson_adam_step(
            ptr(coords), ptr(source), args.batch, ptr(boundary), args.boundary, 1.0,
            ptr(params), ptr(exp_avg), ptr(exp_avg_sq), ptr(step), ptr(loss), None, None,
            ptr(ws), size, 1e-4, 0.9, 0.999, 1e-8, 0.0, stream), "step")

    return run


def _event_us(lib: ctypes.CDLL, run, calls: int) -> float:
    """Median per-call time of `run` with `lib`, HIP events around each call."""
    for _ in range(3):
        run(lib)
    times = []
    for _ in range(calls):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        run(lib)
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3)
    return statistics.median(times)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("workload", choices=["step", "backward"])
    ap.add_argument("--batch", type=int, default=16384)
    ap.add_argument("--boundary", type=int, default=1024)
    ap.add_argument("--calls", type=int, default=20)
    ap.add_argument("--compare", action="store_true",
                    help="also time the library build's call with HIP events")
    ap.add_argument("--by-xcd", action="store_true",
                    help="also print the last call's wave start and end times and shader clock "
                         "per XCD (workgroup index mod 8: the dispatcher deals workgroups to the "
                         "8 XCDs round-robin)")
    args = ap.parse_args(argv)
    if args.workload == "backward":
        args.boundary = 0
    print(f"# phase clock: {args.workload}, batch {args.batch}, boundary {args.boundary}, "
          f"{args.calls} calls", flush=True)
    lib = _load(CLOCK_LIBRARY)
    shape = [ctypes.c_int(), ctypes.c_int(), ctypes.c_int()]
    lib.fhoad_phase_clock_shape(*(ctypes.byref(v) for v in shape))
    workgroups, waves, fields = (v.value for v in shape)
    if fields != FIELDS:
        raise SystemExit(f"the library's table has {fields} fields, this script reads {FIELDS}")
    run = _workload(args)
    table = (ctypes.c_ulonglong * (workgroups * waves * fields))()
    for _ in range(3):
        run(lib)
    per_call = []  # per call: list of rows (one per wave that ran)
    for _ in range(args.calls):
        _check(lib, lib.fhoad_phase_clock_reset(), "phase clock reset")
        run(lib)
        _check(lib, lib.fhoad_phase_clock_read(table), "phase clock read")
        rows = [table[i * fields:(i + 1) * fields] for i in range(workgroups * waves)]
        last_by_workgroup = [(i // waves, r) for i, r in enumerate(rows) if r[WALL_END] != 0]
        per_call.append([r for r in rows if r[WALL_END] != 0])
    waves_run = len(per_call[0])

    def med(values):
        return statistics.median(values)

    # Per call: mean over waves of each phase's cycles; clock rate from cycles / wall time.
    mhz = med([
        statistics.mean(sum(r[:len(PHASES)]) / ((r[WALL_END] - r[WALL_START]) / WALL_MHZ)
                        for r in rows)
        for rows in per_call])
    span_us = med([(max(r[WALL_END] for r in rows) - min(r[WALL_START] for r in rows)) / WALL_MHZ
                   for rows in per_call])
    tiles = med([statistics.mean(r[TILES] for r in rows) for rows in per_call])
    btiles = med([statistics.mean(r[BOUNDARY_TILES] for r in rows) for rows in per_call])
    print(f"\n{waves_run} waves; mean 64-point tiles per wave {tiles:.2f}, boundary tiles per wave "
          f"{btiles:.2f}; shader clock {mhz:.0f} MHz (cycles / s_memrealtime); instrumented "
          f"kernel span {span_us:.1f} us (first wave start to last wave end)")
    if args.compare:
        base = _load(LIBRARY)
        print(f"library build, whole call with HIP events: {_event_us(base, run, args.calls):.1f} us; "
              f"measurement build: {_event_us(lib, run, args.calls):.1f} us")
    print("\n| phase | what | cycles per wave (mean) | us per wave | cycles per 64-point tile |")
    print("|---|---|---:|---:|---:|")
    total = 0.0
    for i, (name, what) in enumerate(PHASES):
        cyc = med([statistics.mean(r[i] for r in rows) for rows in per_call])
        total += cyc
        per_tile = f"{cyc / tiles:,.0f}" if tiles and name not in ("stage", "boundary", "partials", "rest") else ""
        print(f"| {name} | {what} | {cyc:,.0f} | {cyc / mhz:.2f} | {per_tile} |")
    print(f"| total | | {total:,.0f} | {total / mhz:.2f} | |")
    # The spread of wave end times shows the imbalance of the persistent grid.
    ends = sorted(med_end for med_end in (
        (r[WALL_END] - min(q[WALL_START] for q in per_call[-1])) / WALL_MHZ for r in per_call[-1]))
    q = lambda f: ends[min(len(ends) - 1, int(f * len(ends)))]  # noqa: E731
    print(f"\nwave end times of the last call (us after the first start): min {ends[0]:.1f}, "
          f"median {q(0.5):.1f}, 90% {q(0.9):.1f}, max {ends[-1]:.1f}")
    if btiles:
        with_b = [r for r in per_call[-1] if r[BOUNDARY_TILES]]
        without = [r for r in per_call[-1] if not r[BOUNDARY_TILES]]
        for label, rows in (("with a boundary tile", with_b), ("without", without)):
            if rows:
                end = statistics.mean((r[WALL_END] - r[WALL_START]) / WALL_MHZ for r in rows)
                print(f"waves {label}: {len(rows)}, mean wave time {end:.1f} us")
    if args.by_xcd:
        t0 = min(r[WALL_START] for _, r in last_by_workgroup)
        print("\nper XCD, last call (us after the first wave's start; clock = a wave's cycles over "
              "its wall time):\n")
        print("| XCD | waves | start | end (min / median / max) | shader clock MHz (median) |")
        print("|---|---:|---|---|---:|")
        for xcd in range(8):
            rows = [r for wg, r in last_by_workgroup if wg % 8 == xcd]
            if not rows:
                continue
            starts = [(r[WALL_START] - t0) / WALL_MHZ for r in rows]
            ends = sorted((r[WALL_END] - t0) / WALL_MHZ for r in rows)
            clocks = [sum(r[:len(PHASES)]) / ((r[WALL_END] - r[WALL_START]) / WALL_MHZ) for r in rows]
            print(f"| {xcd} | {len(rows)} | {min(starts):.1f}-{max(starts):.1f} | {ends[0]:.1f} / "
                  f"{statistics.median(ends):.1f} / {ends[-1]:.1f} | {statistics.median(clocks):.0f} |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
