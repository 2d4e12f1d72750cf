#!/usr/bin/env python3
"""Benchmark of the MI355X neighbor-list hot path (one JSON line on stdout).

Headline workload (the north-star target): C4, a
100,000-atom periodic float32 box of 100 A edge, cutoff 6 A, cell_list,
quantities 'PD'.  One step is one public ``neighbor_list`` call with the
inputs already resident in HBM (count pass, one host read of E, emit pass).
``value`` is whole-job throughput in M pairs/s.

Also reported:
  roofline      the dominant kernel (the cell-list emit kernel) timed with
                HIP events on the stream it runs on, launched back to back
                into two output sets in turn; achieved = algorithmic bytes
                per launch (N*3*4 + E*(16+12)) / average duration, against
                the 8 TB/s MI355X HBM peak (the interval in its place in the
                request, behind the count, is reported beside it)
  kernel_sum    count pipeline + emit timed the same way (no host gaps)
  cpu_baseline  the reference CPU core (oracle/_ref, when built) or the
                oracle restatement, on the full C4 workload with every
                host core, median of 7 calls
  secondary     C2 (batched crystals, the metric's second workload), C3 and
                C5 measured the same way as the headline (no CPU leg)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "pairs/sec (M edges/s) + achieved HBM GB/s, 100k-atom box and batched crystals"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def to_device(cfg, dev):
    import torch

    return {
        "positions": torch.as_tensor(cfg["positions"]).to(dev),
        "cell": torch.as_tensor(cfg["cell"]).to(dev),
        "pbc": torch.as_tensor(cfg["pbc"]).to(dev),
        "batch_ptr": torch.as_tensor(cfg["batch_ptr"]).to(dev),
    }


def public_call(cfg, t):
    from tonari_amd import neighbor_list

    return neighbor_list(
        cfg["quantities"], t["positions"], t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"],
        algorithm=cfg["algorithm"], sorted=cfg["sorted"], half_list=cfg["half_list"],
        include_self=cfg["include_self"],
    )


def time_public(cfg, t, steps: int, warmup: int):
    """Wall time of `steps` public calls bracketed by device synchronisation."""
    import torch

    out = None
    for _ in range(warmup):
        out = public_call(cfg, t)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = public_call(cfg, t)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    n_pairs = int(out[0].shape[0]) if out else 0
    del out
    return elapsed / steps, n_pairs


def time_phases(cfg, t, reps: int):
    """HIP-event durations of the count pipeline and of the emit kernel.

    Drives the C ABI as a repeated call of the frontend does, on torch's
    current stream: events around tnr_count_async and around the tnr_emit
    queued right behind it, one request per repetition, with the hit-mask
    rows the frontend gives a repeat (the first, untimed repetition's
    reported width plus one).  For a cell-list
    workload tnr_emit launches one kernel (the cell-list emit), so the second
    interval is that kernel's duration in its place in the request.
    """
    import torch

    from tonari_amd._extensions import ALGORITHMS, Outputs, Request, load_torch_hip
    from tonari_amd._torch_frontend import _mask_words

    lib = load_torch_hip()
    pos = t["positions"]
    dev = pos.device
    req = Request(
        dtype=0 if pos.dtype == torch.float32 else 1, algorithm=ALGORITHMS[cfg["algorithm"]],
        n_atoms=pos.shape[0], n_structures=t["batch_ptr"].numel() - 1,
        positions=pos.data_ptr(), batch_ptr=t["batch_ptr"].data_ptr(),
        cell=t["cell"].data_ptr(), pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"],
        half_list=int(cfg["half_list"]), include_self=int(cfg["include_self"]),
        sorted=int(cfg["sorted"]), stencil_reach=0,
    )
    ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    host = torch.empty(8, dtype=torch.int64, pin_memory=True)
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream(dev).cuda_stream
    count_ms, emit_ms = [], []
    quantities = cfg["quantities"]
    n = ctypes.c_int64(0)
    outs = []
    o = None
    for rep in range(reps + 1):
        # one request as the product runs it: the counting pipeline (with the
        # previous repetition's plan as its hint), then the emitting pass
        # queued right behind it (no host wait in between; the inputs do not
        # change, so E, the plan and the bins are the previous repetition's
        # and are checked afterwards)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record()
        hint = o[0].plan if o is not None else -1
        rc = lib.tnr_count_async_hinted(ctypes.byref(req), ws.data_ptr(), ws_bytes,
                                        host.data_ptr(), stream, hint, err, len(err))
        ev[1].record()
        if rc == 0 and o is not None:
            # two output sets in turn, as in the timed loop of the public call
            # (the previous call's outputs are still held while the next runs)
            rc = lib.tnr_emit(ctypes.byref(req), ws.data_ptr(), ws_bytes,
                              ctypes.byref(o[rep % 2]), stream, err, len(err))
        ev[2].record()
        torch.cuda.synchronize()
        if rc != 0 or lib.tnr_count_finish(host.data_ptr(), ctypes.byref(n), err, len(err)) != 0:
            raise RuntimeError(err.value.decode())
        E = int(n.value)
        if o is None:  # the first repetition sizes the outputs and warms caches
            dt = pos.dtype
            shapes = {"P": ((E, 2), torch.int64), "S": ((E, 3), torch.int32),
                      "i": ((E,), torch.int64), "j": ((E,), torch.int64),
                      "d": ((E,), dt), "D": ((E, 3), dt)}
            # hit-mask rows as the frontend sizes a repeat: the width this
            # count reported, plus one
            req.mask_words = _mask_words(int(host[5]))
            ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            o = []
            for _ in range(2):
                out = {q: torch.empty(shapes[q][0], dtype=shapes[q][1], device=dev)
                       for q in set(quantities)}
                ptr = lambda q: out[q].data_ptr() if q in out else None  # noqa: E731
                outs.append(out)
                o.append(Outputs(n_pairs=E, plan=int(host[3]), n_tasks=int(host[4]),
                                 pairs=ptr("P"), shifts=ptr("S"), distances=ptr("d"),
                                 vectors=ptr("D"), sources=ptr("i"), targets=ptr("j")))
            continue
        if (E, int(host[3]), int(host[4])) != (o[0].n_pairs, o[0].plan, o[0].n_tasks):
            raise RuntimeError("the count changed between repetitions of the same input")
        count_ms.append(ev[0].elapsed_time(ev[1]))
        emit_ms.append(ev[1].elapsed_time(ev[2]))
    plan = int(host[3])
    # the emitting pass alone, `reps` launches back to back into the two
    # output sets in turn on the same workspace (the emit can run again on
    # it): each launch's duration with only the gap between two emits, as a
    # kernel trace averages it, where the interval above also holds the
    # transition from the count's last kernel
    emit_alone_ms = None
    if o is not None:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record()
        for rep in range(reps):
            rc = lib.tnr_emit(ctypes.byref(req), ws.data_ptr(), ws_bytes,
                              ctypes.byref(o[rep % 2]), stream, err, len(err))
            if rc != 0:
                raise RuntimeError(err.value.decode())
        ev[1].record()
        torch.cuda.synchronize()
        emit_alone_ms = ev[0].elapsed_time(ev[1]) / reps
    del outs, ws
    return statistics.mean(count_ms), statistics.mean(emit_ms), E, plan, emit_alone_ms


def measured_peak(nbytes: int, reps: int = 20):
    """Measured write and copy bandwidth of plain device kernels.

    A fill of `nbytes` (torch's fill kernel: writes only, the emit's traffic
    pattern) into two buffers in turn, as the bench's emit alternates two
    output sets (the previous fill's dirty lines are still being written back
    from the memory-attached last-level cache while the next one runs), and a
    device-to-device copy of `nbytes` (reads and writes, 2 * nbytes moved).
    HIP events on the current stream; mean over `reps` launches after one
    warm-up launch of each buffer.
    """
    import torch

    dev = torch.device("cuda:0")
    words = nbytes // 4
    bufs = [torch.empty(words, dtype=torch.int32, device=dev) for _ in range(2)]
    src = torch.ones(words, dtype=torch.int32, device=dev)

    def timed(fn):
        for k in range(2):
            fn(k)
        torch.cuda.synchronize()
        ts = []
        for k in range(reps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record()
            fn(k)
            ev[1].record()
            torch.cuda.synchronize()
            ts.append(ev[0].elapsed_time(ev[1]) * 1e-3)
        return statistics.mean(ts), min(ts)

    fill_mean, fill_min = timed(lambda k: bufs[k % 2].fill_(k))
    same_mean, _ = timed(lambda k: bufs[0].fill_(k))
    copy_mean, _ = timed(lambda k: bufs[k % 2].copy_(src))
    del bufs, src
    nb = words * 4
    return {
        "fill_alternating_GBps": round(nb / fill_mean / 1e9, 1),
        "fill_alternating_best_GBps": round(nb / fill_min / 1e9, 1),
        "fill_same_buffer_GBps": round(nb / same_mean / 1e9, 1),
        "copy_GBps": round(2 * nb / copy_mean / 1e9, 1),
        "bytes": nb,
        "method": "torch fill_ of int32 into two buffers in turn (writes only), the same into "
                  "one buffer, and copy_ between buffers (read + write); HIP events, mean of "
                  f"{reps} launches",
    }


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        data = json.load(fh)
    return data.get("hbm_bytes_per_launch")


def time_backward(cfg, t, reps: int):
    """The gradient of sum(w * D) for positions and cell, three ways.

    - fused_us: the autograd backward of the public call's D (positions and
      cell requiring grad), which runs tnr_geometry_backward, with torch's
      allocations and zero fills around it;
    - kernel_us: tnr_geometry_backward alone, HIP events on the stream it
      runs on, with its algorithmic bytes and roofline fraction
      (per pair: P 16 B, S 12 B and dL/dD 3s read; per atom: the position
      gradient 3s written);
    - torch_index_add_us: a fair Torch restatement of the same gradient:
      index_add_ of dL/dD into the targets and of -dL/dD into the sources
      (sources come sorted), and the cell gradient as S^T @ dL/dD (one
      structure);
    - torch_expression_us: autograd of the reference's Torch expression for D
      (``_torch_frontend.py:92-104``), whose scatter-adds of the cell
      gradient all land in the one cell.
    """
    import torch

    from tonari_amd._extensions import load_torch_hip
    from tonari_amd._torch_frontend import _torch_geometry

    positions = t["positions"].clone().requires_grad_()
    cell = t["cell"].clone().requires_grad_()
    P, S, D = public_call(dict(cfg, quantities="PSD"), dict(t, positions=positions, cell=cell))
    w = torch.randn(D.shape, dtype=D.dtype, device=D.device)
    result = {}

    def events(fn, n_rep):
        times = []
        for rep in range(n_rep + 1):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record()
            fn()
            ev[1].record()
            torch.cuda.synchronize()
            if rep > 0:
                times.append(ev[0].elapsed_time(ev[1]) * 1e3)
        return round(statistics.median(times), 2)

    loss = (w * D).sum()
    result["fused_us"] = events(
        lambda: torch.autograd.grad(loss, (positions, cell), retain_graph=True), reps)

    lib = load_torch_hip()
    pos_d, cell_d = positions.detach(), cell.detach()
    gp = torch.zeros_like(pos_d)
    gc = torch.zeros_like(cell_d)
    Dd = D.detach()
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream(pos_d.device).cuda_stream
    nb = t["batch_ptr"].numel() - 1

    def kernel():
        rc = lib.tnr_geometry_backward(
            0 if pos_d.dtype == torch.float32 else 1, P.shape[0], pos_d.shape[0], nb,
            t["batch_ptr"].data_ptr(), P.data_ptr(), S.data_ptr(), Dd.data_ptr(), None,
            w.data_ptr(), None, gp.data_ptr(), gc.data_ptr(), stream, err, len(err))
        if rc != 0:
            raise RuntimeError(err.value.decode())

    result["kernel_us"] = events(kernel, reps)
    s = pos_d.element_size()
    b_alg = P.shape[0] * (16 + 12 + 3 * s) + pos_d.shape[0] * 3 * s + nb * 9 * s
    result["algorithmic_bytes"] = int(b_alg)
    result["kernel_GBps"] = round(b_alg / (result["kernel_us"] * 1e-6) / 1e9, 1)
    result["kernel_frac"] = round(result["kernel_GBps"] / HBM_PEAK_GBPS, 4)

    src, dst = P[:, 0], P[:, 1]
    Sf = S.to(pos_d.dtype)

    def index_add():
        g_pos = torch.zeros_like(pos_d)
        g_pos.index_add_(0, dst, w)
        g_pos.index_add_(0, src, w, alpha=-1)
        g_cell = (Sf.t() @ w).unsqueeze(0)
        return g_pos, g_cell

    result["torch_index_add_us"] = events(index_add, reps)
    # both restatements agree with the fused kernel (checked once, loosely:
    # float atomics sum in varying order)
    g_pos, g_cell = index_add()
    gp.zero_()
    gc.zero_()
    kernel()
    torch.cuda.synchronize()
    scale = float(g_pos.abs().max()) + 1.0
    result["index_add_matches"] = bool(torch.allclose(gp, g_pos, rtol=1e-3, atol=1e-4 * scale)
                                       and torch.allclose(gc, g_cell, rtol=1e-3,
                                                          atol=1e-4 * float(g_cell.abs().max())))
    # the Torch expression takes seconds on C4 (its scatter-adds into the one
    # cell contend): one timed repetition after the warm-up
    D_torch = _torch_geometry(positions, cell, t["batch_ptr"], P, S)
    loss_t = (w * D_torch).sum()
    result["torch_expression_us"] = events(
        lambda: torch.autograd.grad(loss_t, (positions, cell), retain_graph=True), 1)
    result["n_pairs"] = int(P.shape[0])
    return result


def cpu_quantities(quantities, positions, cell, batch_ptr, pairs, shifts):
    """The reference frontend's assembly of i/j/d/D, on CPU tensors.

    Restates ``src/tonari/_torch_frontend.py:78-105`` (bucketize of the
    sources into structures, gathers, einsum of S with the cells, vector
    norm), so the CPU baseline's "public call" variant pays what the
    reference's public CPU call pays after its native search.
    """
    import torch

    values = {"P": pairs, "S": shifts}
    source, target = pairs[:, 0], pairs[:, 1]
    if "i" in quantities:
        values["i"] = source.contiguous()
    if "j" in quantities:
        values["j"] = target.contiguous()
    if "d" in quantities or "D" in quantities:
        pair_batch = torch.bucketize(source.contiguous(), batch_ptr[1:], right=True)
        values["D"] = positions[target] - positions[source] + torch.einsum(
            "ei,eij->ej", shifts.to(positions.dtype), cell[pair_batch])
        if "d" in quantities:
            values["d"] = torch.linalg.vector_norm(values["D"], dim=1)
    return tuple(values[q] for q in quantities)


def time_cpu(fn, warmup_s: float, budget_s: float, min_reps: int = 3, max_reps: int = 7):
    """Warm up for at least warmup_s (at least one call), then repeat until max_reps
    samples or budget_s elapsed (at least min_reps); median of the samples.

    The method of ``benchmarks/run_cpu_benchmark.py:120-161`` (time-based warm-up,
    median of repeats), with the repeats bounded by time.
    """
    t0 = time.perf_counter()
    warm = 0
    while warm == 0 or time.perf_counter() - t0 < warmup_s:
        out = fn()
        warm += 1
        del out
    samples = []
    t1 = time.perf_counter()
    while len(samples) < max_reps and (len(samples) < min_reps or
                                       time.perf_counter() - t1 < budget_s):
        s = time.perf_counter()
        out = fn()
        samples.append(time.perf_counter() - s)
        del out
    return statistics.median(samples), len(samples), warm


def cpu_baseline(name, cfg, mode: str, budget_s: float = 8.0):
    """The reference CPU path on the same workload, with every host core.

    Two variants (the north star's CPU baseline): the native search alone
    (P and S, as the reference's CPU provider returns them), and the public
    call, which also assembles the configuration's quantities from P and S
    with torch on the CPU as the reference frontend does.  The native search
    is the reference's own CPU core built from its sources (oracle/_ref) when
    present, else this repository's restatement of it (oracle/).
    """
    import torch

    import oracle

    kind = "reference" if mode in ("auto", "reference") and oracle.available("reference") else "port"
    if mode == "reference" and kind != "reference":
        log("oracle/_ref is not built; using the restatement")
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    positions = torch.from_numpy(cfg["positions"])
    cell = torch.from_numpy(cfg["cell"])
    batch_ptr = torch.from_numpy(cfg["batch_ptr"])
    algorithm = cfg["algorithm"]

    def native():
        return oracle.neighbor_pairs(
            cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"],
            half_list=cfg["half_list"], include_self=cfg["include_self"],
            algorithm=algorithm, threads=cores, kind=kind)

    def public():
        P, S = native()
        return cpu_quantities(cfg["quantities"], positions, cell, batch_ptr,
                              torch.from_numpy(P), torch.from_numpy(S))

    pairs = len(native()[0])
    res = {"unit": "M pairs/s", "cores": cores, "kind": kind, "n_pairs": pairs}
    for variant, fn in (("native_PS", native), ("public", public)):
        med, reps, warm = time_cpu(fn, 1.0, budget_s)
        res[variant] = {"value": round(pairs / med / 1e6, 3), "ms_per_call": round(med * 1e3, 3),
                        "repeats": reps, "warmup_calls": warm}
    res["value"] = res["native_PS"]["value"]
    res["sample"] = (f"full {name} workload ({len(cfg['positions'])} atoms, {pairs} pairs, "
                     f"algorithm {algorithm}); native_PS = P+S from the CPU search with "
                     f"{cores} threads, public = the same plus '{cfg['quantities']}' assembled "
                     f"with torch ({cores} threads); >= 1 s warm-up, median of the repeats")
    return res


def boundary_report(cfg, t, width: float = 1e-5, chunk: int = 1 << 24):
    """Pairs whose distance lies within `width` of the cutoff, on either side.

    The search runs once more with the cutoff widened by 2 * width.  For every
    pair found, the float64 distance decides nearness (|d - rc| < width), and
    the reference's public predicate evaluated in the input type
    (``csrc/core/neighbors_cpu.cpp:247-261``: D accumulated per axis, every
    product and sum rounded, d^2 < (T)(rc^2)) decides whether the pair belongs
    to the list at the real cutoff: `kept` pairs are in it, `excluded` ones
    are not.  These are the pairs whose membership depends on rounding; the
    parity tests compare them bit for bit like every other pair.
    """
    import torch

    from tonari_amd import neighbor_list

    rc = cfg["cutoff"]
    P, S = neighbor_list(
        "PS", t["positions"], t["cell"], t["pbc"], rc + 2 * width, t["batch_ptr"],
        algorithm=cfg["algorithm"], half_list=cfg["half_list"],
        include_self=cfg["include_self"])
    pos, cell = t["positions"], t["cell"]
    T = pos.dtype
    cut2 = torch.tensor(rc * rc, dtype=torch.float64).to(T).to(pos.device)
    bounds = t["batch_ptr"][1:].contiguous()
    near = kept = 0
    for lo in range(0, P.shape[0], chunk):
        p, s = P[lo:lo + chunk], S[lo:lo + chunk]
        b = torch.bucketize(p[:, 0].contiguous(), bounds, right=True)
        c = cell[b]
        ps, pt = pos[p[:, 0]], pos[p[:, 1]]
        D64 = (pt.double() - ps.double() + torch.bmm(s.double().unsqueeze(1),
                                                     c.double().contiguous()).squeeze(1))
        is_near = (torch.linalg.vector_norm(D64, dim=1) - rc).abs() < width
        comp = pt - ps
        for a in range(3):
            comp = comp + s[:, a:a + 1].to(T) * c[:, a, :]
        d2 = comp[:, 0] * comp[:, 0]
        d2 = d2 + comp[:, 1] * comp[:, 1]
        d2 = d2 + comp[:, 2] * comp[:, 2]
        near += int(is_near.sum())
        kept += int((is_near & (d2 < cut2)).sum())
    del P, S
    return {"width_A": width, "pairs_within": near, "kept": kept, "excluded": near - kept,
            "dtype": str(T).replace("torch.", "")}


def time_first_call(cfg, t, reps: int = 5):
    """Wall time of a public call whose request shape has no previous count.

    The frontend then counts, waits for E and emits into exact-size outputs
    (the reference's own sequence); repeated calls of one shape instead queue
    the emit behind the count (what the timed loop measures).
    """
    import torch

    from tonari_amd import _torch_frontend as F

    times = []
    for _ in range(reps + 1):
        F._speculation().clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = public_call(cfg, t)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        del out
    return round(statistics.median(times[1:]) * 1e3, 4)


def sweep_cases():
    """Batches of equal structures for the brute-force / cell-list crossover.

    Periodic cubic cells at density 0.1 /A^3 (rc 6 A) and 0.05 /A^3 (rc 8 A,
    more images per structure), skewed triclinic cells (angles 75, 105, 65
    degrees, C2's kind of crystal) at density 0.1 /A^3 and rc 6 A, and
    non-periodic Gaussian clusters (rc 5 A), from 4 to 2,048 atoms per
    structure, denser around the crossovers; about 16,384 atoms per batch.
    """
    import numpy as np

    from tonari_amd import workloads as W

    rng = np.random.Generator(np.random.PCG64(2027))
    sizes = (4, 8, 16, 32, 48, 64, 80, 96, 112, 128, 160, 192, 256, 512, 1024, 2048)
    for rc, rho, angles in ((6.0, 0.1, None), (8.0, 0.05, None), (6.0, 0.1, (75.0, 105.0, 65.0))):
        for n in sizes:
            B = max(1, 16384 // n)
            if angles is None:
                edge = (n / rho) ** (1.0 / 3.0)
                cell = edge * np.eye(3)
            else:
                unit = W.triclinic_cell((1.0, 1.0, 1.0), angles)
                cell = unit * (n / rho / abs(np.linalg.det(unit))) ** (1.0 / 3.0)
            frac = [rng.uniform(0.0, 1.0, size=(n, 3)) for _ in range(B)]
            pos = [f @ cell for f in frac]
            cfg = W._pack(pos, [cell] * B, [np.ones(3, bool)] * B, [n] * B,
                          np.float32, rc, quantities="PS", algorithm="auto", half_list=False,
                          include_self=False, sorted=False)
            dual = np.linalg.inv(cell)
            reps = [int(np.ceil(rc * np.linalg.norm(dual[:, a]))) for a in range(3)]
            images = int(np.prod([2 * r + 1 for r in reps]))
            kind = "cubic" if angles is None else "triclinic"
            yield f"periodic {kind} rho {rho} rc {rc}", n, B, images, cfg
    for n in (16, 32, 64, 128, 192, 256, 320, 384, 448, 512, 1024, 2048):
        B = max(1, 16384 // n)
        pos = [W._gaussian_molecule(rng, n, sigma=0.5 * n ** (1.0 / 3.0) + 1.0, dmin=0.9)
               for _ in range(B)]
        cfg = W._pack(pos, [np.zeros((3, 3))] * B, [np.zeros(3, bool)] * B, [n] * B,
                      np.float32, 5.0, quantities="PS", algorithm="auto", half_list=False,
                      include_self=False, sorted=False)
        yield "molecules rc 5.0", n, B, 1, cfg


def auto_sweep(dev, steps: int, warmup: int) -> None:
    """Public-call time of brute_force and cell_list on sweep_cases(), one JSON line each."""
    for family, n, B, images, cfg in sweep_cases():
        t = to_device(cfg, dev)
        res = {"family": family, "atoms_per_structure": n, "structures": B, "images": images,
               "N_times_images": n * images}
        for algorithm in ("brute_force", "cell_list"):
            ms, pairs = time_public(dict(cfg, algorithm=algorithm), t, steps, warmup)
            res[f"ms_{algorithm}"] = round(ms * 1e3, 4)
            res["pairs"] = pairs
        res["faster"] = min(("brute_force", "cell_list"), key=lambda a: res[f"ms_{a}"])
        ms_auto, _ = time_public(dict(cfg, algorithm="auto"), t, steps, warmup)
        res["ms_auto"] = round(ms_auto * 1e3, 4)
        print(json.dumps(res), flush=True)
        del t


def measure(name, cfg, steps, warmup, reps, dev, extras: bool = False):
    """GPU timings of one configuration; with `extras`, also its boundary-pair
    report and its first-call latency."""
    from tonari_amd import workloads as W

    t = to_device(cfg, dev)
    ms_step, n_pairs = time_public(cfg, t, steps, warmup)
    count_ms, emit_ms, E, plan, emit_alone_ms = time_phases(cfg, t, reps)
    assert E == n_pairs
    itemsize = cfg["positions"].dtype.itemsize
    b_alg = W.algorithmic_bytes(len(cfg["positions"]), n_pairs, cfg["quantities"], itemsize)
    kernel_sum = count_ms + emit_ms
    res = {
        "n_atoms": len(cfg["positions"]),
        "n_pairs": n_pairs,
        "ms_per_step": round(ms_step * 1e3, 4),
        "M_pairs_per_s": round(n_pairs / ms_step / 1e6, 3),
        "M_atoms_per_s": round(len(cfg["positions"]) / ms_step / 1e6, 3),
        "algorithmic_bytes": b_alg,
        "count_us": round(count_ms * 1e3, 2),
        "emit_us": round(emit_ms * 1e3, 2),
        "emit_alone_us": round(emit_alone_ms * 1e3, 2) if emit_alone_ms else None,
        "kernel_sum_us": round(kernel_sum * 1e3, 2),
        "GBps_kernel_sum": round(b_alg / (kernel_sum * 1e-3) / 1e9, 1),
        "frac_kernel_sum": round(b_alg / (kernel_sum * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "GBps_end_to_end": round(b_alg / ms_step / 1e9, 1),
        "plan": plan,
    }
    if extras:
        res["ms_first_call"] = time_first_call(cfg, t)
        res["boundary"] = boundary_report(cfg, t)
    del t
    return res


# The configurations of BASELINE.json as bench lines: C1 (the reference's
# CPU-runnable case) in both of its algorithms, then C2, C3 and C5.
SECONDARY = {
    "C1": lambda W: W.c1(),
    "C1_cell": lambda W: dict(W.c1(), algorithm="cell_list"),
    "C2": lambda W: W.c2(),
    "C3": lambda W: W.c3(),
    "C5": lambda W: W.c5(),
}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=20, help="event-timed repetitions")
    ap.add_argument("--cpu-baseline", default="auto", choices=["auto", "reference", "port", "off"])
    ap.add_argument("--secondary", default="C1,C1_cell,C2,C3,C5",
                    help="comma list, or 'none'")
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of timed repeats per configuration and CPU variant")
    ap.add_argument("--backward", default="on", choices=["on", "off"],
                    help="also time the C4 backward of D (fused and Torch expression)")
    ap.add_argument("--secondary-only", action="store_true",
                    help="time only the --secondary configurations (one JSON object per line; "
                         "for profiling them) instead of the benchmark line")
    ap.add_argument("--auto-sweep", action="store_true",
                    help="time brute_force against cell_list on batches of equal structures of "
                         "4 to 2,048 atoms (one JSON line per case) instead of the benchmark line")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run a plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path: run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from tonari_amd import workloads as W

    if not os.path.exists(os.path.join(ROOT, "tonari_amd", "_lib", "libtonari_hip.so")):
        from tonari_amd import build

        build.build()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_calibration_mb > 0:
        # A plain device copy of known size: rocprofv3 --pmc reads its
        # FETCH_SIZE / WRITE_SIZE to calibrate the traffic counters.
        nbytes = args.copy_calibration_mb << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {nbytes} bytes read and written per copy")
        del src, dst

    if args.auto_sweep:
        auto_sweep(dev, max(5, args.steps // 2), 3)
        return 0

    names = [s for s in args.secondary.split(",") if s and s != "none"]
    if args.secondary_only:
        for name in names:
            log(f"{name}: timing")
            res = measure(name, SECONDARY[name](W), args.steps, args.warmup, args.reps, dev)
            print(json.dumps({"config": name, **res}), flush=True)
        return 0

    cfg = W.c4()
    log("C4: timing")
    head = measure("C4", cfg, args.steps, args.warmup, args.reps, dev, extras=True)
    log(f"C4: {head}")
    secondary = {}
    for name in names:
        log(f"{name}: timing")
        scfg = SECONDARY[name](W)
        steps = max(3, args.steps // 3) if name == "C5" else args.steps
        secondary[name] = measure(name, scfg, steps, 2, max(3, args.reps // 4), dev, extras=True)
        log(f"{name}: {secondary[name]}")
    backward = None
    if args.backward == "on":
        log("C4: backward of D")
        backward = time_backward(cfg, to_device(cfg, dev), max(3, args.reps // 4))
        log(f"C4 backward: {backward}")
    base = None
    if args.cpu_baseline != "off":
        log("cpu baseline: C4")
        base = cpu_baseline("C4", cfg, args.cpu_baseline, args.cpu_budget)
        log(f"cpu baseline C4: {base}")
        for name in names:
            log(f"cpu baseline: {name}")
            secondary[name]["cpu_baseline"] = cpu_baseline(name, SECONDARY[name](W),
                                                           args.cpu_baseline, args.cpu_budget)
            log(f"cpu baseline {name}: {secondary[name]['cpu_baseline']}")

    log("measured peak: fill and copy")
    peak = measured_peak(head["algorithmic_bytes"])
    log(f"measured peak: {peak}")
    # the emit's average launch duration: back to back, as the kernel trace
    # averages it (the in-request interval, which also holds the transition
    # from the count's last kernel, is reported beside it)
    emit_s = (head["emit_alone_us"] or head["emit_us"]) * 1e-6
    achieved = head["algorithmic_bytes"] / emit_s / 1e9
    in_request = head["algorithmic_bytes"] / (head["emit_us"] * 1e-6) / 1e9
    peak_fill = peak["fill_alternating_GBps"]
    line = {
        "metric": METRIC,
        "value": head["M_pairs_per_s"],
        "unit": "M pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy PCG64, BASELINE.json configs)",
        "config": {
            "workload": "C4: 100000 atoms uniform in a 100 A periodic cube (density 0.1/A^3), "
                        "float32, cutoff 6 A, cell_list, quantities 'PD', full list",
            "n_atoms": head["n_atoms"],
            "n_pairs": head["n_pairs"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_cell_emit<float, 0, false>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": load_traffic("c4_emit"),
            "algorithmic_bytes_per_launch": head["algorithmic_bytes"],
            "avg_launch_us": round(emit_s * 1e6, 2),
            "avg_launch_how": "HIP events around back-to-back launches into two output sets "
                              "in turn on the launch stream",
            "in_request_us": head["emit_us"],
            "in_request_frac": round(in_request / HBM_PEAK_GBPS, 4),
            # the whole request (every kernel of the count and the emit, no
            # host gaps) against the same algorithmic bytes
            "call_kernel_sum_us": head["kernel_sum_us"],
            "call_frac": head["frac_kernel_sum"],
            # the second denominator: a plain fill of the same bytes into
            # alternating buffers on this GPU
            "peak_measured": peak_fill,
            "frac_measured": round(achieved / peak_fill, 4),
            "call_frac_measured": round(head["GBps_kernel_sum"] / peak_fill, 4),
            "peak_measured_detail": peak,
        },
        "cpu_baseline": base,
        "M_atoms_per_s": head["M_atoms_per_s"],
        "kernel_sum_us": head["kernel_sum_us"],
        "count_us": head["count_us"],
        "frac_kernel_sum": head["frac_kernel_sum"],
        "GBps_end_to_end": head["GBps_end_to_end"],
        "ms_first_call": head["ms_first_call"],
        "boundary": head["boundary"],
        "secondary": secondary,
        "backward_C4": backward,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
