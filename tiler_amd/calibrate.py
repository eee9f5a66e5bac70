"""Work-span calibration of the saturated-parallel-fold-steps cost row.

The reference fits its one decision-relevant machine quantity from a
dispatch sweep of the sum family's three strategies
(spikes/program-planning/reduction-dispatch-crossover/README.md:110-140;
consumed by tiler-compiler/src/measured_cost.rs:1-120, declared by
tiler-compiler/src/target/builder.rs:1369 declare_measured_saturated_parallel_fold_steps):

    cost = sum over stages of ( encoder + max(work / P, depth) * step )

where a stage's `work` is its fold steps summed over every invocation and
`depth` its longest sequential path.  P is the fold steps the device retires
at once when saturated; only P moves a decision (encoder and step scale
every candidate alike to first order).

Here the three strategies are this library's own realizations of
strict-serial-sum-f32 over [rows, extent]:
  * serial   tiler_sum_f32_serial: one invocation per row folds the row;
  * split    tiler_sum_f32_partials + serial: P_s = 2^floor(log2(extent)/2)
             partitions of extent / P_s, then a serial fold of the partials;
  * tree     one 256-thread workgroup per row (tiler_sum_f32_rows), or for
             one row the grid tree (tiler_sum_f32_grid + _final): per thread
             a fold of ceil(extent/256) (or n/(256 G)) steps, then the
             in-workgroup combine (a 6-level butterfly and 4 wave partials).
Each cell is timed with HIP events on the context stream (median of
`repeats` back-to-back launches after a warm-up), the cells are split into a
fit set and a held-out set (checkerboard over the grid), and (encoder, P,
step) are fitted by least squares on log cost: a grid over P (2^(1/8)
steps) with the best non-negative (encoder, step) for each P.

`python -m tiler_amd.calibrate` runs the full sweep on device 0 and prints
the table and the fit as Markdown (the form kept under profiles/).
"""
from __future__ import annotations

import math
import sys
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L

COMBINE_STEPS = 6 + 4  # the butterfly's levels and the four wave partials
COMBINE_WORK = 256 * 6 + 4


@dataclass
class Cell:
    rows: int
    extent: int
    seconds: dict = field(default_factory=dict)  # strategy -> measured seconds
    fit_set: bool = True


def split_partitions(extent: int) -> int:
    return 1 << (max(extent, 1).bit_length() - 1) // 2


def stages(strategy: str, rows: int, extent: int, tree_workgroups: int) -> list[tuple[float, float]]:
    """(work, depth) per launch of one strategy on one cell."""
    n = rows * extent
    if strategy == "serial":
        return [(n, extent)]
    if strategy == "split":
        p = split_partitions(extent)
        return [(n, extent // p), (rows * p, p)]
    if rows == 1:  # the grid tree
        g = tree_workgroups
        return [(n + g * COMBINE_WORK, math.ceil(n / (256 * g)) + COMBINE_STEPS),
                (g + COMBINE_WORK, math.ceil(g / 256) + COMBINE_STEPS)]
    return [(rows * (extent + COMBINE_WORK), math.ceil(extent / 256) + COMBINE_STEPS)]


STRATEGIES = ("serial", "split", "tree")


def predict(params: tuple[float, float, float], st: list[tuple[float, float]]) -> float:
    encoder, p, step = params
    return sum(encoder + max(w / p, d) * step for w, d in st)


def _launch(ctx, strategy, x, rows, extent, out):
    if strategy == "serial":
        ctx.sum_f32(x, rows, extent, out, topology=L.SUM_SERIAL)
    elif strategy == "split":
        p = split_partitions(extent)
        ctx.sum_f32(x, rows, extent, out, topology=L.SUM_MULTIPASS, partitions=p, per_partition=extent // p)
    else:
        ctx.sum_f32(x, rows, extent, out, topology=L.SUM_TREE)


def measure(ctx, grid, repeats: int = 5) -> list[Cell]:
    """Times every strategy on every (rows, extent) of `grid`."""
    cells = []
    largest = max(r * e for r, e in grid)
    x = ctx.to_device(np.random.default_rng(0).uniform(-1, 1, largest).astype(np.float32))
    out = ctx.alloc(4 * max(r for r, _ in grid))
    start, stop = ctx.event(), ctx.event()
    try:
        for i, (rows, extent) in enumerate(grid):
            cell = Cell(rows, extent)
            for strategy in STRATEGIES:
                _launch(ctx, strategy, x, rows, extent, out)  # warm: code, caches, workspace
                times = []
                for _ in range(repeats):
                    ctx.record(start)
                    _launch(ctx, strategy, x, rows, extent, out)
                    ctx.record(stop)
                    ctx.synchronize()
                    times.append(ctx.elapsed_ms(start, stop) * 1e-3)
                cell.seconds[strategy] = float(np.median(times))
            cells.append(cell)
    finally:
        ctx.destroy_event(start)
        ctx.destroy_event(stop)
        x.free()
        out.free()
    assign_sets(cells)
    return cells


def assign_sets(cells: list[Cell]) -> None:
    """Checkerboard over the grid's (rows, extent) lattice positions."""
    rows = sorted({c.rows for c in cells})
    extents = sorted({c.extent for c in cells})
    for c in cells:
        c.fit_set = (rows.index(c.rows) + extents.index(c.extent)) % 2 == 0


def fit(cells: list[Cell], tree_workgroups) -> tuple[float, float, float]:
    """Least squares on log cost over the fit set: (encoder, P, step)."""
    rows = [(c, s) for c in cells if c.fit_set for s in STRATEGIES]
    best = None
    for k in range(6 * 8, 26 * 8 + 1):
        p = 2.0 ** (k / 8)
        # cost = encoder * stages + step * sum max(work/P, depth): relative least squares
        a = np.array([[len(stages(s, c.rows, c.extent, tree_workgroups(c.rows * c.extent))),
                       sum(max(w / p, d) for w, d in stages(s, c.rows, c.extent,
                                                              tree_workgroups(c.rows * c.extent)))]
                      for c, s in rows], float)
        m = np.array([c.seconds[s] for c, s in rows])
        coef, *_ = np.linalg.lstsq(a / m[:, None], np.ones(len(m)), rcond=None)
        coef = np.maximum(coef, 1e-12)
        err = float(np.sum(np.log((a @ coef) / m) ** 2))
        if best is None or err < best[0]:
            best = (err, (float(coef[0]), p, float(coef[1])))
    return best[1]


TIE = 1.05  # a verdict whose strategy measures within 5% of the best is right either way


def decisions(cells: list[Cell], params, tree_workgroups, fit_set: bool) -> dict:
    """Serial-or-parallel verdict agreement, and the worst measured penalty
    of a wrong verdict, on one of the two sets.  Where the chosen strategy
    measures within TIE of the best (a tie on the device), the verdict
    agrees whichever side it names."""
    agree = total = 0
    worst = 1.0
    for c in cells:
        if c.fit_set != fit_set:
            continue
        pred = {s: predict(params, stages(s, c.rows, c.extent, tree_workgroups(c.rows * c.extent)))
                for s in STRATEGIES}
        chosen = min(pred, key=pred.get)
        best = min(c.seconds, key=c.seconds.get)
        total += 1
        if (chosen == "serial") == (best == "serial") or c.seconds[chosen] <= TIE * c.seconds[best]:
            agree += 1
        else:
            worst = max(worst, c.seconds[chosen] / c.seconds[best])
    return {"cells": total, "agreed": agree, "worst_penalty": worst}


DEFAULT_GRID = [(r, e) for r in (1, 16, 256, 4096, 65536) for e in (4, 64, 1024, 16384, 262144)
                if r * e <= (1 << 26)]


def calibrate(ctx, grid=None, repeats: int = 5) -> dict:
    grid = grid or DEFAULT_GRID
    cells = measure(ctx, grid, repeats)
    params = fit(cells, ctx.sum_tree_workgroups)
    return {"cells": cells, "encoder_seconds": params[0], "saturated_parallel_fold_steps": params[1],
            "step_seconds": params[2],
            "fit": decisions(cells, params, ctx.sum_tree_workgroups, True),
            "held_out": decisions(cells, params, ctx.sum_tree_workgroups, False)}


def markdown(result: dict, device: str, tree_workgroups) -> str:
    params = (result["encoder_seconds"], result["saturated_parallel_fold_steps"], result["step_seconds"])
    lines = [f"Device: {device}", "",
             "| rows | extent | set | serial (us) | split (us) | tree (us) | measured best | predicted best |",
             "| ---: | ---: | --- | ---: | ---: | ---: | --- | --- |"]
    for c in result["cells"]:
        pred = {s: predict(params, stages(s, c.rows, c.extent, tree_workgroups(c.rows * c.extent)))
                for s in STRATEGIES}
        lines.append(f"| {c.rows} | {c.extent} | {'fit' if c.fit_set else 'held-out'} | "
                     + " | ".join(f"{c.seconds[s] * 1e6:.2f}" for s in STRATEGIES)
                     + f" | {min(c.seconds, key=c.seconds.get)} | {min(pred, key=pred.get)} |")
    lines += ["", "| parameter | fitted |", "| --- | ---: |",
              f"| encoder_seconds | {result['encoder_seconds']:.3e} |",
              f"| saturated_parallel_fold_steps (P) | {result['saturated_parallel_fold_steps']:.4g} |",
              f"| step_seconds | {result['step_seconds']:.3e} |", "",
              "| serial or parallel | cells | agreed | worst penalty when wrong |", "| --- | ---: | ---: | ---: |"]
    for name in ("fit", "held_out"):
        d = result[name]
        lines.append(f"| {name.replace('_', '-')} | {d['cells']} | {d['agreed']} | {d['worst_penalty']:.2f}x |")
    return "\n".join(lines)


def main(argv=None) -> int:
    import tiler_amd

    ctx = tiler_amd.Context(0)
    try:
        print(f"[calibrate] {len(DEFAULT_GRID)} cells x {len(STRATEGIES)} strategies", file=sys.stderr, flush=True)
        result = calibrate(ctx)
        env = ctx.environment
        print(markdown(result, f"{env['device_name']} {env['gcn_arch_name']} CUs={env['compute_units']}",
                       ctx.sum_tree_workgroups))
    finally:
        ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
