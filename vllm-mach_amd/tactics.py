"""Measured per-shape GEMM tactics: the packaged table, its registration, and the sweep
that measures it.

The reference registers a measured table of per-(M, N, K) projection configs with its
native library before warmup and graph capture, after checking the table's config ABI
against the library's (``prepare``, src/vllm_mach/mxfp6/moe_projection.py:35-105, table
src/vllm_mach/mxfp6/profile/qwen35_moe_projection.json, called from
src/vllm_mach/mxfp6/warmup.py:110-112).  Here the table covers the dense GEMMs of this
package (MXFP8, W6A8 and block-FP8): each entry names the tuning fields of
``mxl_gemm_options`` (kernel, splits, tile_n, tile_m, hybrid, waves) that ran fastest at
one exact (M, N, K, weight format, block) shape on an MI355X, next to the time of the
cost model's own choice, and ``prepare`` registers them (``mxl_set_gemm_config``).  A
call at a registered shape whose options leave the tuning automatic then runs the
measured plan; every other shape keeps the cost model.

``tune`` is the sweep that made the packaged table: it times the automatic plan and
every admissible candidate at each shape with the weights rotated over up to 2 GiB of
copies (cold HBM for the larger weights), each candidate as a HIP graph of back-to-back
launches, and keeps the fastest.  Run it on the GPU with::

    python -c "import __graft_entry__ as g; g.load_package().tactics.main()" --out table.json
"""
from __future__ import annotations

import argparse
import datetime
import json
from pathlib import Path
from typing import Iterable, Optional

import torch

from . import _lib, ops

TABLE = Path(__file__).with_name("profile") / "mi355x_gemm_tactics.json"
FIELDS = ("kernel", "splits", "tile_n", "tile_m", "hybrid", "waves")
KERNEL_NAMES = {0: "stream", 1: "wide", 2: "generic", 4: "chunk"}

# The shapes the packaged table was measured on: the benchmark configurations' prefill
# and decode sizes, and the reference's own table shapes (W6A8 projections of the
# reference's MoE model at its measured M values).
BENCH_SHAPES = (
    [(m, 2048, 2048, ops.E4M3, 0) for m in (16, 32, 64, 128, 256, 512)]
    + [(m, 2560, 9216, ops.E4M3, 0) for m in (16, 32, 64, 128, 256, 512)]
    + [(m, 18432, 2560, ops.E4M3, 1) for m in (16, 32, 64, 128, 256, 512)]
    + [(m, 17408, 5120, ops.E2M3, 0) for m in (16, 32, 64, 128, 256)]
)
REFERENCE_SHAPES = [
    (m, n, k, ops.E2M3, 0)
    for (n, k), ms in {
        (512, 2048): (32, 36, 40, 48, 56, 64, 72, 80, 96, 112, 128),
        (2048, 256): (64, 80, 96, 112, 128, 160),
        (2048, 2048): (32, 36, 64, 72, 80, 96, 112, 128),
        (4608, 2048): (32, 72, 80, 96, 112, 128),
        (6144, 2048): (32, 36, 72, 80, 96, 160),
    }.items()
    for m in ms
]


def load_table(path: Optional[Path] = None) -> dict:
    return json.loads(Path(path or TABLE).read_text())


def options_of(config: dict) -> _lib.GemmOptions:
    """The ``mxl_gemm_options`` of a table entry's config (epilogue fields at their defaults)."""
    return _lib.GemmOptions(0, *(int(config[f]) for f in FIELDS))


def _problem_keys(problems) -> set:
    """{(N, K, w_fmt, block)} of ``warmup.collect_problems``-style dense keys
    (kernel class name, N, K, format, dual sizes)."""
    keys = set()
    for cls, n, k, fmt, *_ in problems:
        block = int(cls == "BlockFp8LinearKernel")
        keys.add((int(n), int(k), ops.E4M3 if block else int(fmt), block))
    return keys


def prepare(problems: Optional[Iterable] = None, table=None, mode: str = "auto",
            device: Optional[torch.device] = None) -> int:
    """Register the table's entries with the library; returns how many.

    ``problems``: only entries whose (N, K, format, block) a prepared layer has
    (``warmup.collect_problems(model)[0]`` keys); None registers every entry.  ``table``:
    a path or a loaded table (default: the packaged one).  ``mode``: "off" registers
    nothing, "auto" skips a table measured on a device with another CU count, "on"
    raises instead of skipping.  A table whose config ABI differs from the library's
    raises (the reference's w6a8_config_abi check)."""
    if mode not in ("auto", "on", "off"):
        raise ValueError("mode must be auto, on or off")
    if mode == "off":
        return 0
    t = table if isinstance(table, dict) else load_table(table)
    abi = _lib.query("mxl_gemm_config_abi")
    if t["config_abi"] != abi:
        raise RuntimeError(f"GEMM tactic table config ABI {t['config_abi']!r} does not match the library's {abi!r}")
    dev = None
    if torch.cuda.is_available():
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        if cus != t["cu_count"]:
            if mode == "on":
                raise RuntimeError(f"GEMM tactic table measured on {t['cu_count']} CUs, this device has {cus}")
            return 0
    keys = None if problems is None else _problem_keys(problems)
    count = 0
    # the library keys an entry by the device current at registration
    with torch.cuda.device(dev) if dev is not None else _no_device():
        for e in t["entries"]:
            if keys is not None and (e["n"], e["k"], e["w_fmt"], e["block"]) not in keys:
                continue
            _lib.call("mxl_set_gemm_config", e["m"], e["n"], e["k"], e["w_fmt"], e["block"],
                      _lib.options_ptr(options_of(e["config"])))
            count += 1
    return count


class _no_device:
    """Host-only planning (no HIP device): entries register under device 0."""

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def clear() -> None:
    """Drop every registered entry: the cost model plans every shape again."""
    _lib.call("mxl_clear_gemm_configs")


def installed() -> int:
    return int(_lib.query("mxl_gemm_config_count"))


def plan_name(m: int, n: int, k: int, w_fmt: int, block: int, config: Optional[dict] = None) -> str:
    """The kernels a call at this shape launches (with ``config``'s tuning fields, or the
    current plan: a registered entry or the cost model)."""
    return _lib.plan_name("mxl_gemm_plan_name", m, n, k, w_fmt, block,
                          options=None if config is None else options_of(config))


# ------------------------------------------------------------------------- the sweep

def candidates(m: int, n: int, k: int, w_fmt: int, block: int) -> list[dict]:
    """Tuning fields worth timing at one shape: every kernel the shape admits, and the wide
    kernel over tile widths, K splits, wave counts and the hybrid schedule."""
    base = dict(kernel=-1, splits=0, tile_n=0, tile_m=0, hybrid=0, waves=0)
    out = [dict(base, kernel=kern) for kern in (0, 2, 4)]
    out += [dict(base, kernel=2, splits=s) for s in (1, 2, 4, 8)]
    for nt in (1, 2, 4):
        for s in (1, 2, 3, 4, 6, 8):
            for w in (4, 8):
                out.append(dict(base, kernel=1, tile_n=nt, splits=s, waves=w))
                if s == 1:
                    out.append(dict(base, kernel=1, tile_n=nt, splits=1, waves=w, hybrid=1))
        if m <= 64:
            for s in (1, 2, 4, 8):
                out.append(dict(base, kernel=1, tile_n=nt, tile_m=4, splits=s, waves=4))
    return out


class _Problem:
    """Weights (rotated copies over about 2 GiB, at most 64 of them) and inputs of one
    (N, K, format, block)."""

    def __init__(self, n: int, k: int, w_fmt: int, block: int, dev: torch.device, gen: torch.Generator):
        self.n, self.k, self.w_fmt, self.block = n, k, w_fmt, block
        if block:
            codes = torch.randint(0, 0x7E, (n, k), generator=gen, device=dev, dtype=torch.uint8)
            tiled, _ = ops.pack_weight(codes.view(torch.float8_e4m3fn), None, ops.E4M3)
            self.scale = torch.full(((n + 127) // 128, k // 128), 1e-3, device=dev, dtype=torch.float32)
            copies = min(64, max(2, (2 << 30) // tiled.numel()))
            self.copies = [(tiled.clone(), self.scale) for _ in range(copies)]
        else:
            width = k if w_fmt == ops.E4M3 else k * 3 // 4
            codes = torch.randint(0, 0x7E, (n, width), generator=gen, device=dev, dtype=torch.uint8)
            if w_fmt == ops.E4M3:
                codes = codes.view(torch.float8_e4m3fn)
            scales = torch.randint(118, 126, (n, k // 32), generator=gen, device=dev, dtype=torch.uint8)
            tiled, tiled_s = ops.pack_weight(codes, scales, w_fmt)
            copies = min(64, max(2, (2 << 30) // (tiled.numel() + tiled_s.numel())))
            self.copies = [(tiled.clone(), tiled_s.clone()) for _ in range(copies)]

    def fns(self, m: int, dev: torch.device, gen: torch.Generator) -> list:
        x = torch.randn(m, self.k, generator=gen, device=dev).bfloat16()
        n, k = self.n, self.k
        if self.block:
            a, sa = torch.ops.mach_amd.quantize_block_fp8(x)
            return [lambda w=w, s=s: torch.ops.mach_amd.block_fp8_gemm(a, sa, w, s, n, k, None) for w, s in self.copies]
        a, sa = torch.ops.mach_amd.quantize_mxfp8(x, ops.FLOOR_CARRY175)
        f = self.w_fmt
        return [lambda w=w, s=s: torch.ops.mach_amd.mx_gemm(a, sa, w, s, n, k, f, None) for w, s in self.copies]


def graph_us(fns: list, stream: torch.cuda.Stream, replays: int = 10, trials: int = 5) -> float:
    """Median µs per launch of ``fns`` captured back to back in one HIP graph."""
    with torch.cuda.stream(stream):
        for fn in fns:
            fn()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for fn in fns:
                fn()
        g.replay()
        stream.synchronize()
        times = []
        for _ in range(trials):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for _ in range(replays):
                g.replay()
            e.record(stream)
            e.synchronize()
            times.append(s.elapsed_time(e) * 1000.0 / replays / len(fns))
    times.sort()
    return times[len(times) // 2]


def tune(shapes: Iterable[tuple], device: Optional[torch.device] = None, log=print) -> dict:
    """Time the automatic plan and every candidate at each (M, N, K, w_fmt, block) shape;
    returns a table (one entry per shape: the fastest config, its time, the automatic
    plan's time and kernels).  Registered entries are cleared first, so that "auto" is
    the cost model's own choice."""
    dev = device or torch.device("cuda", torch.cuda.current_device())
    clear()
    gen = torch.Generator(device=dev).manual_seed(0)
    stream = torch.cuda.Stream(device=dev)
    groups: dict = {}
    for m, n, k, f, b in shapes:
        groups.setdefault((n, k, f, b), []).append(m)
    entries = []
    for (n, k, f, b), ms in groups.items():
        prob = _Problem(n, k, f, b, dev, gen)
        for m in sorted(set(ms)):
            fns = prob.fns(m, dev, gen)
            auto_us = graph_us(fns, stream)
            best, best_us = None, auto_us
            for cfg in candidates(m, n, k, f, b):
                try:
                    with ops.tuning(kernel=cfg["kernel"], splits=cfg["splits"], tile_n=cfg["tile_n"],
                                    tile_m=cfg["tile_m"], hybrid=bool(cfg["hybrid"]), waves=cfg["waves"]):
                        us = graph_us(fns, stream)
                except (_lib.MxlError, RuntimeError):
                    continue  # the shape does not admit this kernel or split
                if us < best_us:
                    best, best_us = cfg, us
            if best is None:  # the cost model's plan was fastest: record it as its own entry
                best = dict(kernel=-1, splits=0, tile_n=0, tile_m=0, hybrid=0, waves=0)
            e = dict(m=m, n=n, k=k, w_fmt=f, block=b, config=best, us=round(best_us, 2), auto_us=round(auto_us, 2),
                     plan=plan_name(m, n, k, f, b, best), auto_plan=plan_name(m, n, k, f, b))
            entries.append(e)
            log(f"M={m} N={n} K={k} fmt={f} block={b}: auto {auto_us:.2f} us ({e['auto_plan']}) -> "
                f"{best_us:.2f} us ({e['plan']})", flush=True)
        del prob
        torch.cuda.empty_cache()
    props = torch.cuda.get_device_properties(dev)
    return {
        "config_abi": int(_lib.query("mxl_gemm_config_abi")),
        "device": props.name,
        "cu_count": props.multi_processor_count,
        "measured": datetime.date.today().isoformat(),
        "method": "HIP graph of back-to-back launches over weight copies rotated across 2 GiB (at most 64 "
                  "copies: weights under 32 MiB stay partly in the Infinity Cache); median of 5 trials of 10 "
                  "replays; per-launch microseconds",
        "entries": entries,
    }


def main(argv: Optional[list] = None) -> None:
    ap = argparse.ArgumentParser(description="Measure the per-shape GEMM tactic table on this GPU")
    ap.add_argument("--out", required=True, help="where to write the table (JSON)")
    ap.add_argument("--shapes", choices=("bench", "reference", "all"), default="all")
    args = ap.parse_args(argv)
    shapes = {"bench": BENCH_SHAPES, "reference": REFERENCE_SHAPES,
              "all": BENCH_SHAPES + REFERENCE_SHAPES}[args.shapes]
    table = tune(shapes)
    Path(args.out).write_text(json.dumps(table, indent=1) + "\n")
