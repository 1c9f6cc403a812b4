"""Benchmark of the erasure-coding hot path on one MI355X.

Headline metric: RS(6,3) encode GB/s of data bytes over six 256 MiB shards of
serialized fp32 optimizer state, inputs resident in HBM, and its HBM roofline
fraction.  Also measured in the same run and reported under
"also": RS(6,3) decode with 3 seeded erasures, XOR parity of 4 x 64 MiB bf16
shards, the headline's bytes coded in two other layouts (cut into units, and
stripe-contiguous), the batched configurations, the encode's interference with a GEMM
load, the checkpoint staging path and snapshot saves, a training loop with
periodic saves, and a streaming copy as the practical bandwidth ceiling.  The
CPU baseline is the repo's multithreaded SIMD CPU encoder (the reference ships
none) on a bounded sample of the same bytes.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one encode of the 6 x 256 MiB stripe (one kernel launch).
Prints progress to stderr and one JSON line to stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0   # MI355X published HBM3E bandwidth, GB/s
MiB = 1 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed(fn, steps: int, warmup: int):
    """(wall ms/step, event ms/step) of fn() on torch's current stream,
    bracketed by device synchronisation."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, start.elapsed_time(end) / steps


def settle(fn, seconds: float):
    """Back-to-back calls of fn() on torch's current stream for at least
    `seconds` of wall time, in batches that keep the queue full: the GPU's
    clocks ramp up under sustained load, and a timed region that starts on
    an idle GPU measures the ramp.  Returns (ms spent, calls made)."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(32):
            fn()
        n += 32
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return (time.perf_counter() - t0) * 1e3, n


def steady(fn, steps: int, warmup: int, seconds: float = 0.3):
    """timed() after ``seconds`` of back-to-back calls (settle).  The
    configurations after the headline start right after host-side work (data
    generation, uploads, checks); without the settle their first timed
    launches run on a GPU still raising its clocks (config 5's encode ran
    4.59 ms at the start of a 10-launch window and 4.14 at its end)."""
    settle(fn, seconds)
    return timed(fn, steps, warmup)


def launch_spread(fn, steps: int):
    """Per-launch durations (ms) of `steps` back-to-back calls of fn(), from
    an event pair around each call on torch's current stream: the median
    and extremes next to the timed region's mean."""
    import statistics
    import torch
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return {"median": statistics.median(per), "min": min(per), "max": max(per),
            "mean": ev[0].elapsed_time(ev[-1]) / steps}


def cpu_baseline(shards_np, k: int, m: int, seconds: float, gpu_parity, xor_host, gpu_xor,
                 lost, batched_cpu) -> dict:
    """The repo's multithreaded SIMD CPU encoder (oracle/ec_cpu_fast.c; the
    reference ships none) on bounded samples of the same bytes the GPU coded,
    all usable cores (at most 16, the box's share per GPU) and one core,
    each gated byte for byte against the GPU's output first:
      value   RS(6,3) encode of the first 64 MiB of each 256 MiB shard
              (``seconds`` all-core, a third of that on one core);
      configs XOR 4 x 64 MiB (the whole config), the 3-erasure decode over
              the same 64 MiB samples of the survivors, and the sampled
              stripes of configs 4 and 5 (``batched_cpu``, timed by
              batched_configs while their host bytes exist)."""
    import numpy as np
    import oracle
    sample = [s[: 64 * MiB] for s in shards_np]
    coeff = oracle.cauchy(k, m)
    outs = [np.empty(64 * MiB, np.uint8) for _ in range(m)]
    cores = cpu_cores()
    oracle.fast_rs_encode(coeff, sample, outs, nthreads=cores)
    for i in range(m):
        if not np.array_equal(gpu_parity[i][: 64 * MiB].cpu().numpy(), outs[i]):
            raise AssertionError(f"GPU parity {i} differs from the CPU encoder")
    xor_cpu = oracle.fast_xor_encode(xor_host, nthreads=cores)
    if not np.array_equal(gpu_xor.cpu().numpy(), xor_cpu):
        raise AssertionError("GPU XOR parity differs from the CPU encoder")
    # correctness gate: the baseline must reproduce the scalar oracle
    ref = oracle.rs_encode(coeff, [s[: 1 * MiB] for s in sample])
    chk = oracle.fast_rs_encode(coeff, [s[: 1 * MiB] for s in sample], nthreads=cores)
    if not all(np.array_equal(a, b) for a, b in zip(ref, chk)):
        raise AssertionError("CPU baseline disagrees with the scalar oracle")
    enc = cpu_rates(lambda t: oracle.fast_rs_encode(coeff, sample, outs, nthreads=t),
                    k * 64 * MiB, seconds)
    configs = {}
    xout = np.empty_like(xor_cpu)
    configs["xor_4x64MiB"] = {
        **cpu_rates(lambda t: oracle.fast_xor_encode(xor_host, out=xout, nthreads=t),
                    sum(x.size for x in xor_host), seconds / 5),
        "sample": "the whole config, byte-identical to the GPU parity"}
    # the decode: the GPU recovered the lost shards bit-exactly (checked in
    # main); here the same rows rebuild the 64 MiB samples of the lost shards
    codeword = sample + outs
    surv, rows = oracle.decode_matrix(coeff, k, m, lost)
    rec = [np.empty(64 * MiB, np.uint8) for _ in lost]
    oracle.fast_rs_encode(rows, [codeword[g] for g in surv], rec, nthreads=cores)
    if not all(np.array_equal(r, codeword[g]) for r, g in zip(rec, lost)):
        raise AssertionError("CPU decode does not rebuild the lost shards")
    configs["rs63_decode_3_erasures"] = {
        **cpu_rates(lambda t: oracle.fast_rs_encode(rows, [codeword[g] for g in surv], rec,
                                                    nthreads=t), k * 64 * MiB, seconds / 5),
        "sample": f"lost {list(lost)}: the first 64 MiB of each of the 6 survivors, "
                  "rebuilding the lost shards byte for byte"}
    configs.update(batched_cpu)
    return {
        "value": enc["all_cores_GBps"], "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": (f"RS(6,3) encode of the first 64 MiB of each of the 6 shards "
                   f"(384 MiB data), repeated over ~{seconds:.0f} s with {cores} threads; "
                   f"repo CPU encoder ({oracle.fast_isa()}), the reference ships none"),
        "one_core_GBps": enc["one_core_GBps"],
        "isa": oracle.fast_isa(),
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "configs": configs,
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_cores() -> int:
    """Threads of the CPU baseline: the usable cores, at most 16 (the box's
    share per GPU)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_rates(run, data_bytes: int, seconds: float) -> dict:
    """all-core and one-core GB/s of data for ``run(threads)``, each repeated
    for about ``seconds`` (one core: a third of that) after a warm call."""
    cores = cpu_cores()
    out = {}
    for key, threads, budget in (("all_cores_GBps", cores, seconds),
                                 ("one_core_GBps", 1, seconds / 3)):
        run(threads)
        n, t0 = 0, time.perf_counter()
        while True:
            run(threads)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= budget:
                break
        out[key] = round(n * data_bytes / dt / 1e9, 2)
    out["cores"] = cores
    return out


def cpu_batched(coeff, hptr, hlen, stripes, unit: int, gpu_parity, seconds: float,
                what: str) -> dict:
    """The repo's SIMD CPU encoder (ecfast_encode_batched) over the given
    stripes of a batched layout, through host descriptors of the same bytes
    the GPU coded; gated byte for byte against the GPU's parity of those
    stripes (``gpu_parity``: [len(stripes), m, unit] host array)."""
    import numpy as np
    import oracle
    m = coeff.shape[0]
    dp = np.ascontiguousarray(hptr[stripes])
    dl = np.ascontiguousarray(hlen[stripes])
    par = np.empty((len(stripes), m, unit), np.uint8)
    pp = (np.uint64(par.ctypes.data) +
          np.arange(len(stripes) * m, dtype=np.uint64).reshape(len(stripes), m) * np.uint64(unit))
    run = lambda threads: oracle.fast_encode_batched(coeff, dp, dl, pp, unit, nthreads=threads)
    run(cpu_cores())
    if not np.array_equal(par, gpu_parity):
        raise AssertionError(f"{what}: GPU parity differs from the CPU encoder")
    res = cpu_rates(run, int(dl.sum()), seconds)
    res["sample"] = (f"{len(stripes)} stripes ({int(dl.sum()) / 1e6:.0f} MB of data), "
                     "byte-identical to the GPU parity")
    return res


def cpu_update(lay, changed, host_old, hptr, hlen, par_before, gpu_par, seconds: float) -> dict:
    """The repo's SIMD CPU update (ecfast_parity_update) of config 5's 1 %
    perturbation: every changed stripe, over host descriptors of the new
    bytes (the perturbed host copies), the old bytes (``host_old``, one array
    per changed unit) and a host copy of the parity before the update
    (``par_before``); gated byte for byte against the GPU's updated parity of
    those stripes.  GB/s of changed data and ms per update."""
    import numpy as np
    import torch
    import oracle
    k, m, unit = lay.k, lay.m, lay.unit_bytes
    stripe = changed // k
    st, inv = np.unique(stripe, return_inverse=True)
    nptr = np.zeros((st.size, k), np.uint64)
    optr = np.zeros((st.size, k), np.uint64)
    dl = np.zeros((st.size, k), np.uint32)
    for n, (r, j) in enumerate(zip(inv, changed % k)):
        nptr[r, j] = hptr[stripe[n], j]
        optr[r, j] = host_old[n].ctypes.data
        dl[r, j] = hlen[stripe[n], j]
    par = np.ascontiguousarray(par_before[st])
    pp = (np.uint64(par.ctypes.data) +
          np.arange(st.size * m, dtype=np.uint64).reshape(st.size, m) * np.uint64(unit))
    oracle.fast_parity_update(lay.coeff, nptr, optr, dl, pp, unit, nthreads=cpu_cores())
    idx = torch.as_tensor(st.astype(np.int64), device=gpu_par.device)
    if not np.array_equal(par, gpu_par[idx].cpu().numpy()):
        raise AssertionError("config 5 update: GPU parity differs from the CPU update")
    changed_bytes = int(dl.sum())
    # each further run folds the same delta in again (timing only)
    res = cpu_rates(lambda t: oracle.fast_parity_update(lay.coeff, nptr, optr, dl, pp, unit,
                                                        nthreads=t), changed_bytes, seconds)
    res["all_cores_ms"] = round(changed_bytes / (res["all_cores_GBps"] * 1e9) * 1e3, 3)
    res["one_core_ms"] = round(changed_bytes / (res["one_core_GBps"] * 1e9) * 1e3, 3)
    res["sample"] = (f"the whole update: {changed.size} changed units in {st.size} stripes "
                     f"({changed_bytes / 1e6:.0f} MB of changed data; GB/s of changed data), "
                     "byte-identical to the GPU's updated parity")
    return res


def cpu_decode_batched(lay, views, lost, hptr, hlen, stripes, gpu_parity,
                       seconds: float) -> dict:
    """The repo's SIMD CPU encoder used as a decoder on sampled stripes of
    config 5: the lost positions rebuilt with the decode rows from the k
    survivors (data units through host descriptors of the host copies,
    parity units from a host copy of the GPU's parity of those stripes,
    ``gpu_parity``: [len(stripes), m, unit]); gated byte for byte against the
    host copies of the units (``views``, zero-padded past a short unit's
    end) and the parity.  GB/s of
    data of the sampled stripes, as the GPU's decode rate is quoted."""
    import numpy as np
    import oracle
    k, m, unit = lay.k, lay.m, lay.unit_bytes
    surv, rows = oracle.decode_matrix(lay.coeff, k, m, lost)
    ns = len(stripes)
    dp = np.ascontiguousarray(hptr[stripes])
    dl = np.ascontiguousarray(hlen[stripes])
    gp = np.ascontiguousarray(gpu_parity)
    sp = np.zeros((ns, k), np.uint64)
    sl = np.zeros((ns, k), np.uint32)
    for t, g in enumerate(surv):
        if g < k:
            sp[:, t], sl[:, t] = dp[:, g], dl[:, g]
        else:
            sp[:, t] = (np.uint64(gp.ctypes.data) + np.arange(ns, dtype=np.uint64)
                        * np.uint64(m * unit) + np.uint64((g - k) * unit))
            sl[:, t] = unit
    e = len(lost)
    out = np.empty((ns, e, unit), np.uint8)
    op = (np.uint64(out.ctypes.data) +
          np.arange(ns * e, dtype=np.uint64).reshape(ns, e) * np.uint64(unit))
    run = lambda threads: oracle.fast_encode_batched(rows, sp, sl, op, unit, nthreads=threads)
    run(cpu_cores())
    for r, g in enumerate(lost):
        if g >= k:
            ok = np.array_equal(out[:, r], gp[:, g - k])
        else:
            ok = True
            for n, s in enumerate(stripes):
                want = np.zeros(unit, np.uint8)
                u = s * k + g
                if u < lay.n_units:
                    t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
                    piece = views[t][i * unit: (i + 1) * unit]
                    want[: piece.size] = piece
                ok &= np.array_equal(out[n, r], want)
        if not ok:
            raise AssertionError(f"config 5 CPU decode does not rebuild position {g}")
    res = cpu_rates(run, int(dl.sum()), seconds)
    res["sample"] = (f"lost {list(lost)}: {ns} stripes ({int(dl.sum()) / 1e6:.0f} MB of data), "
                     "rebuilding the lost units and parity byte for byte")
    return res


def batched_configs(pkg, synth, dev, seed: int, gemm: "GemmLoad", cpu_seconds: float = 0.0,
                    with_checkpoint: bool = True) -> dict:
    """Configs 4 and 5 through the batched stripe launcher: data GB/s of one
    launch (HIP events) and HBM traffic GB/s, with product-only checks (a
    decode round trip; update == full re-encode).  The bytes are drawn on
    the host (numpy, seeded, on the box's cores) and uploaded; with
    ``cpu_seconds`` the repo's CPU encoder is timed on sampled stripes of the
    same host bytes (key "cpu").  ``with_checkpoint`` adds the checkpoint
    staging and snapshot measurements on config 5's tensors."""
    import numpy as np
    import torch
    from megatron_lm_amd.layout import stripe_descriptors
    out, cpu = {}, {}
    # config 4: one rank's 20.8 GB buffer, RS(8,2), 4 MiB units (620 stripes)
    t0 = time.perf_counter()
    host = synth.gpt_rank_buffer_host(seed)
    t1 = time.perf_counter()
    buf = torch.from_numpy(host).to(dev)
    torch.cuda.synchronize()
    log(f"config 4: {host.size / 1e9:.2f} GB drawn in {t1 - t0:.1f} s, uploaded in "
        f"{time.perf_counter() - t1:.1f} s")
    lay = pkg.StripeLayout([buf], 8, 2, 4 * MiB)
    par = lay.alloc_parity()
    w, e = steady(lambda: lay.encode(par), 10, 2)
    if cpu_seconds:
        _, hptr, hlen = stripe_descriptors([host.ctypes.data], [host.size], 8, 4 * MiB)
        sample = list(range(16)) + [lay.n_stripes - 1]
        cpu["rs82_20.8GB"] = {**cpu_batched(lay.coeff, hptr, hlen, sample, 4 * MiB,
                                            par[sample].cpu().numpy(), cpu_seconds,
                                            "config 4"),
                              "gpu_GBps": round(lay.data_bytes / (w * 1e-3) / 1e9, 1)}
        log(f"config 4 CPU: {cpu['rs82_20.8GB']}")
    del host
    keep = (lay.unit_view(3).clone(), par[0, 1].clone())
    lay.unit_view(3).zero_()
    par[0, 1].zero_()
    lay.decode(par, [3, 9], stripes=[0])
    torch.cuda.synchronize()
    if not (torch.equal(lay.unit_view(3), keep[0]) and torch.equal(par[0, 1], keep[1])):
        raise AssertionError("RS(8,2) batched round trip failed")
    out["rs82_20.8GB_GBps"] = round(lay.data_bytes / (w * 1e-3) / 1e9, 1)
    out["rs82_20.8GB_traffic_GBps"] = round((lay.data_bytes + par.numel()) / (e * 1e-3) / 1e9, 1)
    out["rs82_20.8GB_ms"] = round(e, 3)
    log(f"config 4 RS(8,2) {lay.n_stripes} stripes: {out['rs82_20.8GB_GBps']} GB/s data")
    del buf, lay, par, keep
    torch.cuda.empty_cache()

    # config 5: 3,000 ragged tensors, RS(12,4), 64 KiB units, 1% update
    tensors, views = ragged_tensors(synth, dev, seed, with_host=True)
    lay = pkg.StripeLayout(tensors, 12, 4, 64 << 10)
    par = lay.alloc_parity()
    w, e = steady(lambda: lay.encode(par), 10, 2)
    U5 = 64 << 10
    _, hptr, hlen = stripe_descriptors([v.ctypes.data for v in views],
                                       [v.size for v in views], 12, U5)
    sample = list(range(0, lay.n_stripes, max(1, lay.n_stripes // 2000)))
    if cpu_seconds:
        cpu["rs124_ragged"] = {**cpu_batched(lay.coeff, hptr, hlen, sample, U5,
                                             par[sample].cpu().numpy(), cpu_seconds,
                                             "config 5"),
                               "gpu_GBps": round(lay.data_bytes / (w * 1e-3) / 1e9, 1)}
        log(f"config 5 CPU: {cpu['rs124_ragged']}")
    out["rs124_ragged_GBps"] = round(lay.data_bytes / (w * 1e-3) / 1e9, 1)
    out["rs124_ragged_traffic_GBps"] = round((lay.data_bytes + par.numel()) / (e * 1e-3) / 1e9, 1)
    out["rs124_ragged_data_GB"] = round(lay.data_bytes / 1e9, 2)
    log(f"config 5 RS(12,4) {lay.n_units} units: {out['rs124_ragged_GBps']} GB/s data")
    # The seeded 1 % perturbation: new bytes from seeded numpy, written to the
    # device tensors and to the host copies (the old bytes kept on both sides).
    changed = synth.perturbed_units(seed, lay.n_units, 0.01)
    fresh_bytes = synth.perturbation_bytes(seed, lay.host_len.reshape(-1)[changed])
    par_before = par.cpu().numpy() if cpu_seconds else None
    olds, host_old = [], []
    for u, nb in zip(changed.tolist(), fresh_bytes):
        v = lay.unit_view(u)
        olds.append(v.clone())
        v.copy_(torch.from_numpy(nb))
        t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
        hv = views[t][i * U5: i * U5 + nb.size]
        host_old.append(hv.copy())
        hv[:] = nb
    plan = lay.plan_update(par, changed, olds)
    lay.run(plan)
    fresh = lay.encode()
    torch.cuda.synchronize()
    if not torch.equal(par, fresh):
        raise AssertionError("incremental update differs from a full re-encode")
    del fresh
    if cpu_seconds:
        cpu["rs124_update_1pct"] = cpu_update(lay, changed, host_old, hptr, hlen, par_before,
                                              par, cpu_seconds)
        log(f"config 5 update CPU: {cpu['rs124_update_1pct']}")
    del par_before, host_old
    # each further run folds the same delta in again (timing only)
    w, e = steady(lambda: lay.run(plan), 10, 2)
    changed_bytes = int(lay.host_len.reshape(-1)[changed].sum())
    upd_read, upd_write = update_bytes(lay, changed)
    upd_traffic = upd_read + upd_write
    out["update_1pct_changed_GB"] = round(changed_bytes / 1e9, 3)
    out["update_1pct_ms"] = round(e, 3)
    out["update_1pct_traffic_GBps"] = round(upd_traffic / (e * 1e-3) / 1e9, 1)
    if "rs124_update_1pct" in cpu:
        cpu["rs124_update_1pct"]["gpu_ms"] = out["update_1pct_ms"]
    lay.encode(par)  # repeated update runs toggled the parity; restore it
    lost = [1, 7, 12, 14]
    dplan = lay.plan_decode(par, lost)
    w, e = steady(lambda: lay.run(dplan), 5, 1)
    k5, S5 = 12, lay.n_stripes
    surv = [p for p in range(16) if p not in lost][:k5]
    hl = lay.host_len.astype(np.int64)
    dec_traffic = sum(int(hl[:, p].sum()) if p < k5 else S5 * U5 for p in surv + lost)
    out["rs124_ragged_decode4_GBps"] = round(lay.data_bytes / (e * 1e-3) / 1e9, 1)
    out["rs124_ragged_decode4_traffic_GBps"] = round(dec_traffic / (e * 1e-3) / 1e9, 1)
    log(f"update {out['update_1pct_ms']} ms, decode {out['rs124_ragged_decode4_GBps']} GB/s")
    # the same decode kernel by lost set: where the written units lie among the
    # read ones sets the rate (parity only: the tensors are only read)
    by_set = {}
    for other in ([12, 13, 14, 15], [0, 1, 2, 3], [1, 7]):
        oplan = lay.plan_decode(par, other)
        _, eo = steady(lambda: lay.run(oplan), 5, 1)
        osurv = [p for p in range(16) if p not in other][:k5]
        otraffic = sum(int(hl[:, p].sum()) if p < k5 else S5 * U5 for p in osurv + other)
        by_set[",".join(map(str, other))] = round(otraffic / (eo * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)
        del oplan
    by_set["1,7,12,14"] = round(dec_traffic / (e * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)
    out["rs124_ragged_decode_frac_by_lost_set"] = by_set
    log(f"decode, fraction of the roofline by lost set: {by_set}")
    if cpu_seconds:
        cpu["rs124_ragged_decode4"] = {
            **cpu_decode_batched(lay, views, lost, hptr, hlen, sample,
                                 par[sample].cpu().numpy(), cpu_seconds),
            "gpu_GBps": out["rs124_ragged_decode4_GBps"]}
        log(f"config 5 decode CPU: {cpu['rs124_ragged_decode4']}")
    del views, hptr, hlen, olds, plan, dplan
    # the snapshot's kernel: encode plus a zero-padded copy of every data
    # unit into one stripe-major (stripes, 16, 64 KiB) block, one pass over
    # the data
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    block = torch.empty((S5, 16, U5), dtype=torch.uint8, device=dev)
    bp, gp = GpuSliceCodec._unit_ptrs(block, 12, 4), GpuSliceCodec._unit_ptrs(block, 0, 12)
    L, st = pkg._lib.lib(), pkg.codec.stream_handle(None, dev)

    def copy_encode():
        pkg._lib.check(L.ec_encode_batched_copy(
            pkg._lib.u8ptr(lay.coeff), 12, 4, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
            bp.data_ptr(), gp.data_ptr(), S5, U5, st), "ec_encode_batched_copy")
    w, e = steady(copy_encode, 5, 1)
    out["rs124_ragged_copy_encode_traffic_GBps"] = round((lay.data_bytes + block.numel()) /
                                                        (e * 1e-3) / 1e9, 1)
    out["rs124_ragged_copy_encode_ms"] = round(e, 3)
    log(f"copying encode {out['rs124_ragged_copy_encode_traffic_GBps']} GB/s of traffic")
    # The freed blocks stay in torch's cache (no empty_cache here): the
    # staging below reuses them, and returning tens of GB of device memory
    # to the driver right before it slows host <-> device transfers for
    # about 2 s (measured: 40 GB freed with empty_cache, then the same
    # staging call took 0.87 s of transfer time instead of 0.48).
    del lay, par, block, bp, gp
    if with_checkpoint:
        out.update(checkpoint_staging(pkg, tensors))
        out.update(checkpoint_snapshot(pkg, tensors, gemm))
    del tensors
    torch.cuda.empty_cache()
    if cpu:
        out["cpu"] = cpu
    return out


def checkpoint_staging(pkg, tensors) -> dict:
    """The save and load sides of the erasure-coded checkpoint manager on one
    GPU, for config 5's tensors: encode into k + m slices staged to host
    memory through 1 GiB pinned chunks, and back: k slices with two data
    positions missing to rebuilt tensors.  Data GB/s over wall time.  The
    first encode writes a fresh host array (page faults and zeroing on first
    touch: the "cold" rate); each result is handed back with release() and
    the next encode reuses its array, as the manager's repeated saves do.
    The transfers share the host's PCIe and memory with other tenants, so the
    median of three calls is reported for each direction."""
    import statistics
    import torch
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    codec = GpuSliceCodec(12, 4, 64 << 10)
    nbytes = sum(t.numel() * t.element_size() for t in tensors)
    dev = tensors[0].device
    try:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, slices = codec.encode(tensors)
        t_cold = time.perf_counter() - t0
        stats = [codec.last_stage_stats]
        t_enc = []
        for _ in range(3):
            codec.release(slices)            # the next encode writes into the same array
            t0 = time.perf_counter()
            meta, slices = codec.encode(tensors)
            t_enc.append(time.perf_counter() - t0)
            stats.append(codec.last_stage_stats)
        keep = {p: slices[p] for p in range(16) if p not in (2, 9)}  # lose 2 data slices
        keep = dict(list(sorted(keep.items()))[:12])
        t_dec = []
        for _ in range(3):
            t0 = time.perf_counter()
            rebuilt = codec.decode(meta, keep, dev)
            t_dec.append(time.perf_counter() - t0)
            ok = all(torch.equal(a.view(-1).view(torch.uint8), b.view(-1).view(torch.uint8))
                     for a, b in zip(rebuilt, tensors))
            if not ok:
                raise AssertionError("checkpoint decode did not rebuild the tensors")
            del rebuilt
        del keep
        codec.release(slices)
        log(f"staging calls: encode {[round(t, 3) for t in t_enc]} s (cold {t_cold:.3f}), "
            f"decode {[round(t, 3) for t in t_dec]} s")
        for name, st in zip(["cold", "warm 1", "warm 2", "warm 3"], stats):
            log(f"staging {name}: {st}")
        res = {"ckpt_encode_to_host_GBps": round(nbytes / statistics.median(t_enc) / 1e9, 1),
               "ckpt_encode_to_host_cold_GBps": round(nbytes / t_cold / 1e9, 1),
               "ckpt_decode_from_host_GBps": round(nbytes / statistics.median(t_dec) / 1e9, 1),
               "ckpt_encode_calls_s": [round(t, 3) for t in [t_cold] + t_enc],
               "ckpt_encode_stage_stats": stats}
    except RuntimeError as e:  # pinned-memory limits differ between hosts
        res = {"ckpt_staging_error": str(e)[:200]}
    log(f"checkpoint staging: {res}")
    return res


class GemmLoad:
    """A training-like load: 8192^3 bf16 GEMMs on torch's current stream."""
    N = 8192

    def __init__(self, dev):
        import torch
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        self.a = torch.randn(self.N, self.N, device=dev, dtype=torch.bfloat16, generator=g)
        self.b = torch.randn(self.N, self.N, device=dev, dtype=torch.bfloat16, generator=g)
        self.c = torch.empty(self.N, self.N, device=dev, dtype=torch.bfloat16)
        self.flops = 2 * self.N ** 3

    def enqueue(self, n: int):
        """n GEMMs bracketed by timing events on the current stream."""
        import torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            torch.matmul(self.a, self.b, out=self.c)
        e1.record()
        return e0, e1

    def ms_alone(self, n: int = 30) -> float:
        import torch
        self.enqueue(20)   # clocks settle
        torch.cuda.synchronize()
        e0, e1 = self.enqueue(n)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n


def overlap_with_training(pkg, dev, data, parity, coeff, gemm: "GemmLoad") -> dict:
    """Checkpoint encode concurrent with a training-like load: GEMMs on
    torch's stream, the RS(6,3) encode beside them on (a) the engine's side
    stream, which has a hardware queue of its own, and (b) a stream from
    torch's pool, which shares a queue with torch's stream.  Default priority
    both.  The encode is sized to outlast the GEMM window, so the GEMM's time
    per call is measured under load throughout (HIP events on each stream)."""
    import torch
    n_gemm = 60
    g_before = gemm.ms_alone()

    def enc_ms(side, n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        for _ in range(n):
            pkg.matvec(coeff, data, out=parity, stream=side)
        e1.record(side)
        return e0, e1

    out = {}
    g_alone = g_before
    data_bytes = sum(t.numel() for t in data)
    for tag, side in (("", pkg.side_stream(dev)), ("_pooled_stream", torch.cuda.Stream(device=dev))):
        e0, e1 = enc_ms(side, 20)
        torch.cuda.synchronize()
        e_alone = e0.elapsed_time(e1) / 20
        n_enc = max(8, int(1.3 * n_gemm * g_alone / e_alone))
        e0, e1 = enc_ms(side, n_enc)
        g0, g1 = gemm.enqueue(n_gemm)
        torch.cuda.synchronize()
        g_both, e_both = g0.elapsed_time(g1) / n_gemm, e0.elapsed_time(e1) / n_enc
        out[f"overlap_gemm_ms_with_encode{tag}"] = round(g_both, 3)
        out[f"overlap_encode_GBps_alone{tag}"] = round(data_bytes / e_alone / 1e6, 1)
        out[f"overlap_encode_GBps_with_gemm{tag}"] = round(data_bytes / e_both / 1e6, 1)
    # the GEMM's clock drifts by several per cent over a run: alone is the
    # mean of a measurement before and one after the concurrent runs
    g_alone = (g_before + gemm.ms_alone()) / 2
    out["overlap_gemm_ms_alone"] = round(g_alone, 3)
    out["overlap_gemm_TFLOPs_alone"] = round(gemm.flops / g_alone / 1e9, 1)
    log(f"overlap: GEMM {g_alone:.3f} ms alone, {out['overlap_gemm_ms_with_encode']} ms beside "
        f"the encode on the side stream, {out['overlap_gemm_ms_with_encode_pooled_stream']} ms "
        f"on a pooled stream")
    return out


def checkpoint_snapshot(pkg, tensors, gemm: "GemmLoad") -> dict:
    """The save path that keeps training running, for config 5's tensors:
    GpuSliceCodec.snapshot codes them into one HBM block on the side stream
    and holds torch's stream only until that is done (the stall a save costs
    training), then stages the block to host memory in a background thread
    while GEMMs run on torch's stream.  Reports the stall (median of three
    saves, each right after 20 GEMMs have run, as a save follows a training
    step), the staging time to host memory, and the GEMM time per call during
    the last save's staging next to its time alone; the slices are checked
    against the synchronous encode's."""
    import numpy as np
    import torch
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    codec = GpuSliceCodec(12, 4, 64 << 10)
    nbytes = sum(t.numel() * t.element_size() for t in tensors)
    try:
        g_alone = gemm.ms_alone()
        codec.release(codec.snapshot(tensors).result()[1])   # warm: pinned buffers, host array
        stalls = []
        for rep in range(3):
            gemm.enqueue(20)[1].synchronize()   # a training step's GPU work has just ended
            t0 = time.perf_counter()
            pending = codec.snapshot(tensors)
            mark = torch.cuda.Event()
            mark.record()             # torch's stream passes it once the coding is done
            mark.synchronize()
            stalls.append(time.perf_counter() - t0)
            if rep < 2:
                codec.release(pending.result()[1])
        t_stall = sorted(stalls)[1]
        # about 0.25 s of GEMMs, enqueued at once so that no host gap enters
        # their timing, inside the staging (which takes about twice as long)
        n_gemm = max(10, int(0.25 / (g_alone * 1e-3)))
        g0, g1 = gemm.enqueue(n_gemm)
        g1.synchronize()
        contained = not pending.done()
        _, slices = pending.result()
        t_staged = time.perf_counter() - t0
        g_during = g0.elapsed_time(g1) / n_gemm
        _, again = codec.encode(tensors)          # a second host array: slices is alive
        # every parity byte, and the head of every data slice
        if not all(np.array_equal(a, b) for a, b in zip(slices[12:], again[12:])) or \
                not all(np.array_equal(a[:64 << 20], b[:64 << 20])
                        for a, b in zip(slices[:12], again[:12])):
            raise AssertionError("snapshot slices differ from the synchronous encode")
        codec.release(again)
        codec.release(slices)
        del again, slices
        res = {"ckpt_snapshot_stall_ms": round(t_stall * 1e3, 2),
               "ckpt_snapshot_stall_ms_each": [round(x * 1e3, 2) for x in stalls],
               "ckpt_snapshot_stall_data_GBps": round(nbytes / t_stall / 1e9, 1),
               "ckpt_snapshot_staged_s": round(t_staged, 3),
               "ckpt_snapshot_gemm_ms_alone": round(g_alone, 3),
               "ckpt_snapshot_gemm_ms_during_staging": round(g_during, 3),
               "ckpt_snapshot_gemm_calls_during_staging": n_gemm,
               "ckpt_snapshot_gemm_window_inside_staging": contained}
    except RuntimeError as e:  # HBM or pinned-memory limits differ between hosts
        res = {"ckpt_snapshot_error": str(e)[:200]}
    log(f"checkpoint snapshot: {res}")
    return res


def skeleton_ceilings(pkg, dev, shard: int, enc_traffic_gbs: float) -> dict:
    """Practical ceiling of the RS(6,3) access pattern on this box: the RS
    kernel's memory skeleton (libec_probe.so: same loads, stores and tile
    order, the GF arithmetic replaced by one XOR) over 256 MiB streams, with
    6 reads only, 3 writes only, and both.  6 reads and 3 writes run back to
    back would move 9 / (6 / read + 3 / write) bytes per unit time: the bound
    the encode is compared with."""
    import ctypes
    import torch
    path = os.path.join(ROOT, "probe", "libec_probe.so")
    if not os.path.exists(path):
        return {}
    lib = ctypes.CDLL(path)
    lib.ecp_stream.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                               ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    ins = [torch.empty(shard, dtype=torch.uint8, device=dev).random_(0, 256) for _ in range(6)]
    outs = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in range(3)]
    sink = torch.zeros(16, dtype=torch.uint8, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptrs = lambda ts: (ctypes.c_void_p * max(1, len(ts)))(*[t.data_ptr() for t in ts])

    def run(r, w):
        rc = lib.ecp_stream(ptrs(ins[:r]), r, ptrs(outs[:w]), w, shard, sink.data_ptr(), st)
        if rc:
            raise RuntimeError(f"ecp_stream({r}, {w}) returned {rc}")
    out = {}
    for name, r, w in (("read6", 6, 0), ("write3", 0, 3), ("mix63", 6, 3)):
        _, ev = timed(lambda: run(r, w), 50, 10)
        out[name] = (r + w) * shard / (ev * 1e-3) / 1e9
    bound = 9 / (6 / out["read6"] + 3 / out["write3"])
    del ins, outs
    return {"skeleton_read6_GBps": round(out["read6"], 1),
            "skeleton_write3_GBps": round(out["write3"], 1),
            "skeleton_mix63_GBps": round(out["mix63"], 1),
            "mix_bound_GBps": round(bound, 1),
            "encode_frac_of_mix_bound": round(enc_traffic_gbs / bound, 4)}


def stripe_layouts(pkg, dev, data) -> dict:
    """RS(6,3) over config 2's bytes (``data``: 6 x 256 MiB) placed three ways, each
    timed like the headline (clock settle, then HIP events around 50
    back-to-back launches) and checked byte for byte against the flat
    kernel's parity:
      flat          the flat kernel on six separate 256 MiB shards, parity in
                    three separate 256 MiB buffers;
      cut           the batched kernel over the same six shards cut into
                    units (stripe s = the s-th unit of every shard, parity
                    written into the three separate buffers the same way):
                    the flat kernel's access order;
      contiguous    the batched kernel over one 1.5 GiB buffer holding the
                    same units stripe after stripe (the six units of a stripe
                    adjacent, then its three parity units adjacent), the
                    layout the checkpoint path builds from a rank's tensors.
    Fraction of the 8 TB/s roofline from the 9 x 256 MiB of HBM traffic."""
    import numpy as np
    import torch
    k, m, shard = 6, 3, 256 * MiB
    assert len(data) == k and all(d.numel() == shard for d in data)
    coeff = pkg.cauchy_matrix(k, m)
    par = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in range(m)]
    L = pkg._lib.lib()
    st = pkg.codec.stream_handle(None, dev)
    traffic = (k + m) * shard

    def rate(fn):
        settle(fn, 0.3)
        _, ev = timed(fn, 50, 5)
        return {"us": round(ev * 1e3, 1),
                "frac": round(traffic / (ev * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)}

    out = {"flat": rate(lambda: pkg.rs_encode(data, m, out=par))}
    torch.cuda.synchronize()
    for U in (64 << 10, 1 * MiB):
        n = shard // U
        views = [data[j][s * U:(s + 1) * U] for s in range(n) for j in range(k)]
        cut = pkg.StripeLayout(views, k, m, U, coeff)
        cut_par = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in range(m)]
        pp = (np.array([p.data_ptr() for p in cut_par], dtype=np.uint64)[None, :]
              + np.arange(n, dtype=np.uint64)[:, None] * np.uint64(U))
        d_pp = torch.from_numpy(np.ascontiguousarray(pp).view(np.int64)).to(dev)

        def cut_encode():
            pkg._lib.check(L.ec_encode_batched(
                pkg._lib.u8ptr(cut.coeff), k, m, cut.d_ptrs.data_ptr(), cut.d_len.data_ptr(),
                d_pp.data_ptr(), n, U, st), "ec_encode_batched")
        tag = f"{U >> 10}KiB"
        out[f"cut_{tag}"] = rate(cut_encode)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(cut_par, par)):
            raise AssertionError(f"cut layout ({tag} units): parity differs from the flat kernel")
        del cut, cut_par, d_pp, views
        buf = torch.stack([d.view(n, U) for d in data], dim=1).reshape(-1)
        cont = pkg.StripeLayout([buf], k, m, U, coeff)
        cont_par = cont.alloc_parity()
        out[f"contiguous_{tag}"] = rate(lambda: cont.encode(cont_par))
        torch.cuda.synchronize()
        for i in range(m):
            if not torch.equal(cont_par[:, i].reshape(-1), par[i]):
                raise AssertionError(f"contiguous layout ({tag} units): parity {i} differs")
        del buf, cont, cont_par
        torch.cuda.empty_cache()
    del par
    torch.cuda.empty_cache()
    log(f"stripe layouts: {out}")
    return out


def small_shards(pkg, dev) -> dict:
    """RS(6,3) over small shards, where the per-call host work competes with
    the kernel: back-to-back eager calls (matvec into given outputs, and
    rs_encode allocating its parity; each checks its tensors in the torch
    binding on every call) and launches of a ShardPlan (built once, one
    foreign call per launch).  HBM traffic GB/s over wall time, 9 shards per
    call."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    coeff = pkg.cauchy_matrix(6, 3)
    out = {}
    for mib in (1, 4):
        n = mib * MiB
        data = [torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g)
                for _ in range(6)]
        par = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(3)]
        plan = pkg.ShardPlan(coeff, data, out=par)
        calls = 400
        w_eager, _ = timed(lambda: pkg.matvec(coeff, data, out=par), calls, 50)
        w_alloc, _ = timed(lambda: pkg.rs_encode(data, 3), calls, 50)
        w_plan, _ = timed(plan, calls, 50)
        out[f"rs63_{mib}MiB_eager_traffic_GBps"] = round(9 * n / (w_eager * 1e-3) / 1e9, 1)
        out[f"rs63_{mib}MiB_eager_alloc_traffic_GBps"] = round(9 * n / (w_alloc * 1e-3) / 1e9, 1)
        out[f"rs63_{mib}MiB_plan_traffic_GBps"] = round(9 * n / (w_plan * 1e-3) / 1e9, 1)
        out[f"rs63_{mib}MiB_eager_us_per_call"] = round(w_eager * 1e3, 2)
        out[f"rs63_{mib}MiB_eager_alloc_us_per_call"] = round(w_alloc * 1e3, 2)
        out[f"rs63_{mib}MiB_plan_us_per_call"] = round(w_plan * 1e3, 2)
    log(f"small shards: {out}")
    return out


def update_bytes(lay, changed):
    """(read, write) algorithmic bytes of the incremental update of the
    units ``changed``: the new and old bytes of each changed unit, and the m
    parity units of each changed stripe up to the stripe's longest changed
    unit (past it the delta is zero, and the kernel leaves the parity
    alone), read and written back."""
    import numpy as np
    lens = lay.host_len.reshape(-1)[changed].astype(np.int64)
    stripes, inv = np.unique(np.asarray(changed) // lay.k, return_inverse=True)
    longest = np.zeros(stripes.size, np.int64)
    np.maximum.at(longest, inv, lens)
    parity = lay.m * int(longest.sum())
    return 2 * int(lens.sum()) + parity, parity


def ragged_tensors(synth, dev, seed: int, with_host: bool = False):
    """Config 5's 3,000 tensors (bf16 / fp32, log-uniform 4 KiB - 64 MiB),
    drawn on the host (synth.ragged_host) and uploaded one by one; with
    ``with_host`` also their host byte arrays."""
    import torch
    t0 = time.perf_counter()
    block, views, kinds = synth.ragged_host(seed)
    t1 = time.perf_counter()
    tensors = [torch.from_numpy(v).to(dev).view(torch.bfloat16 if kd == 0 else torch.float32)
               for v, kd in zip(views, kinds.tolist())]
    torch.cuda.synchronize()
    log(f"config 5: {block.size / 1e9:.2f} GB drawn in {t1 - t0:.1f} s, uploaded in "
        f"{time.perf_counter() - t1:.1f} s")
    return (tensors, views) if with_host else tensors


def batched_pmc_launches(pkg, synth, dev, seed: int) -> int:
    """Counter-run workload for the batched launcher, three launches each, in
    this order: the engine's streaming copy of one 256 MiB shard (the
    calibration kernel of known traffic); config 5 (RS(12,4), 3,000 ragged
    tensors, 64 KiB units): encode, copying encode into one stripe-major
    (stripes, 16, 64 KiB) block (the snapshot's kernel), decode of lost positions 1, 7, 12,
    14, 1 % update; config 4 (RS(8,2), 20.8 GB buffer, 4 MiB units) encode,
    which the library runs as two kernels per launch (the full tiles and the
    rest).  Prints the launch groups with their algorithmic bytes and kernel
    dispatches as JSON."""
    import numpy as np
    import torch
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    groups = []

    def three(name, fn, read, write, kernels=1):
        torch.cuda.synchronize()
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        groups.append({"name": name, "launches": 3, "dispatches": 3 * kernels,
                       "read_bytes": int(read), "write_bytes": int(write)})

    shard = 256 * MiB
    src = torch.empty(shard, dtype=torch.uint8, device=dev).random_(0, 256)
    dst = torch.empty_like(src)
    three("copy", lambda: pkg.xor_encode([src], out=dst), shard, shard)
    del src, dst
    tensors = ragged_tensors(synth, dev, seed)
    k, m, U = 12, 4, 64 << 10
    lay = pkg.StripeLayout(tensors, k, m, U)
    par = lay.alloc_parity()
    S = lay.n_stripes
    valid = lay.data_bytes
    three("c5_encode", lambda: lay.encode(par), valid, par.numel())
    block = torch.empty((S, k + m, U), dtype=torch.uint8, device=dev)
    pp = GpuSliceCodec._unit_ptrs(block, k, m)
    gp = GpuSliceCodec._unit_ptrs(block, 0, k)
    L = pkg._lib.lib()
    st = pkg.codec.stream_handle(None, dev)

    def copy_encode():
        pkg._lib.check(L.ec_encode_batched_copy(
            pkg._lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
            pp.data_ptr(), gp.data_ptr(), S, U, st), "ec_encode_batched_copy")
    three("c5_copy_encode", copy_encode, valid, block.numel())
    del block, pp, gp
    three("c5_encode_again", lambda: lay.encode(par), valid, par.numel())
    lost = [1, 7, 12, 14]
    dplan = lay.plan_decode(par, lost)
    # survivors: data positions 0, 2-6, 8-11 and parity 13, 15 of every stripe;
    # outputs: the valid bytes of data positions 1 and 7, parity 12 and 14
    surv = [p for p in range(k + m) if p not in lost][:k]
    hl = lay.host_len.astype(np.int64)
    read = sum(int(hl[:, p].sum()) if p < k else S * U for p in surv)
    write = sum(int(hl[:, p].sum()) if p < k else S * U for p in lost)
    three("c5_decode4", lambda: lay.run(dplan), read, write)
    changed = synth.perturbed_units(seed, lay.n_units, 0.01)
    olds = [lay.unit_view(u).clone() for u in changed.tolist()]
    uplan = lay.plan_update(par, changed, olds)
    three("c5_update", lambda: lay.run(uplan), *update_bytes(lay, changed))
    del lay, par, dplan, uplan, olds, tensors
    torch.cuda.empty_cache()
    host = synth.gpt_rank_buffer_host(seed)
    buf = torch.from_numpy(host).to(dev)
    del host
    lay = pkg.StripeLayout([buf], 8, 2, 4 * MiB)
    par = lay.alloc_parity()
    three("c4_encode", lambda: lay.encode(par), lay.data_bytes, par.numel(), kernels=2)
    print(json.dumps({"mode": "batched-pmc", "groups": groups}), flush=True)
    return 0


def measured_traffic(k: int, m: int, shard: int):
    """HBM bytes per RS(6,3) launch from the committed counter summary
    (profiles/rs_encode_6x256MiB_pmc.json: FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by the same counter on a copy of known size), or
    None when it is absent or describes another shape."""
    path = os.path.join(ROOT, "profiles", "rs_encode_6x256MiB_pmc.json")
    try:
        with open(path) as f:
            pmc = json.load(f)
    except (OSError, ValueError):
        return None
    if (k, m, shard) != (6, 3, 256 * MiB) or pmc.get("algorithmic_bytes") != (k + m) * shard:
        return None
    return pmc.get("traffic_bytes")


def pmc_launches(pkg, dev) -> int:
    """Counter-run workload: 3 launches of the engine's streaming copy (XOR
    of one 256 MiB shard: reads 256 MiB, writes 256 MiB, the calibration
    kernel of known traffic), then 3 of the RS(6,3) encode over 6 x 256 MiB,
    then 3 of config 1's XOR(4) over 4 x 64 MiB."""
    import torch
    shard = 256 * MiB
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    data = [torch.randint(0, 256, (shard,), dtype=torch.uint8, device=dev, generator=g)
            for _ in range(6)]
    out = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in range(3)]
    torch.cuda.synchronize()
    for _ in range(3):
        pkg.xor_encode(data[:1], out=out[0])
    torch.cuda.synchronize()
    coeff = pkg.cauchy_matrix(6, 3)
    for _ in range(3):
        pkg.matvec(coeff, data, out=out)
    torch.cuda.synchronize()
    xs = 64 * MiB
    xin = [d[:xs] for d in data[:4]]
    for _ in range(3):
        pkg.xor_encode(xin, out=out[0][:xs])
    torch.cuda.synchronize()
    print(json.dumps({"mode": "pmc", "copy_bytes_read": shard, "copy_bytes_written": shard,
                      "rs_bytes_read": 6 * shard, "rs_bytes_written": 3 * shard,
                      "xor_bytes_read": 4 * xs, "xor_bytes_written": xs}), flush=True)
    return 0


def training_with_checkpoints(pkg, dev, steps: int = 40, every: int = 10) -> dict:
    """A training loop with periodic erasure-coded checkpoints: 8 bf16-autocast
    8192 x 8192 linear layers over 8192 tokens, fp32 parameters with AdamW
    (the checkpointed state: parameters and both moments, 6.4 GB), one step =
    forward, backward, optimizer step.  The same ``steps`` run three times:
    without checkpoints, with a synchronous save (GpuSliceCodec.encode, slices
    in host memory before training resumes) every ``every`` steps, and with a
    snapshot save (GpuSliceCodec.snapshot: training resumes once the state is
    coded in HBM; staging runs in the background).  Reports ms per step of
    each and the save's overhead per save."""
    import torch
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    torch.manual_seed(0)
    n, layers = 8192, 8
    model = torch.nn.Sequential(*[torch.nn.Linear(n, n, bias=False) for _ in range(layers)]).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-5)
    x = torch.randn(n, n, device=dev, dtype=torch.bfloat16)

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(x).float().pow(2).mean()
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=False)

    for _ in range(3):
        step()
    torch.cuda.synchronize()

    def state():
        return [t for p in model.parameters()
                for t in (p.data, opt.state[p]["exp_avg"], opt.state[p]["exp_avg_sq"])]

    nbytes = sum(t.numel() * t.element_size() for t in state())
    codec = GpuSliceCodec(12, 4, 4 << 20)
    pending = []

    def run(save):
        codec.release(codec.snapshot(state()).result()[1])  # warm: host array, pinned buffers
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            step()
            if save == "sync" and (i + 1) % every == 0:
                codec.release(codec.encode(state())[1])   # slices written: array reused
            elif save == "snapshot" and (i + 1) % every == 0:
                if pending:   # the previous save's slices are written by now: hand
                    codec.release(pending.pop().result()[1])   # their array back for reuse
                pending.append(codec.snapshot(state()))
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        for p in pending:
            codec.release(p.result()[1])
        pending.clear()
        return t * 1e3 / steps

    base = run(None)
    sync = run("sync")
    snap = run("snapshot")
    saves = steps // every
    res = {"train_state_GB": round(nbytes / 1e9, 2), "train_steps": steps, "train_save_every": every,
           "train_ms_per_step": round(base, 2),
           "train_ms_per_step_sync_saves": round(sync, 2),
           "train_ms_per_step_snapshot_saves": round(snap, 2),
           "train_ms_per_sync_save": round((sync - base) * steps / saves, 1),
           "train_ms_per_snapshot_save": round((snap - base) * steps / saves, 1)}
    del model, opt, x
    torch.cuda.empty_cache()
    log(f"training with checkpoints: {res}")
    return res


def training_in_child() -> dict:
    """training_with_checkpoints in a child process: a training process
    starts with its own allocator and host memory, not with what the rest
    of this benchmark left behind."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--mode", "train"],
                           capture_output=True, text=True, timeout=300)
        line = [ln for ln in r.stdout.splitlines() if ln.startswith('{"mode": "train"')]
        if r.returncode != 0 or not line:
            return {"train_error": (r.stderr or r.stdout)[-200:]}
        res = json.loads(line[0])
        res.pop("mode")
        return res
    except subprocess.TimeoutExpired:
        return {"train_error": "timed out"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="back-to-back encodes before the warmup and timed steps, so that "
                         "the timed region does not measure the GPU's clock ramp")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batched", action="store_true",
                    help="skip the 20.8 GB RS(8,2) and ragged RS(12,4) configurations")
    ap.add_argument("--mode", choices=["full", "headline", "decode", "flat-kernels", "pmc",
                                       "batched", "batched-kernels", "batched-pmc",
                                       "train", "small-shards", "layout"],
                    default="full",
                    help="full: everything (default); headline: only the timed RS(6,3) "
                         "encode (for kernel-trace profiles); flat-kernels: configs 2, 3 "
                         "and 1 and the streaming-copy ceiling, timed as in full (for "
                         "kernel-trace profiles); pmc: a few launches of a "
                         "plain 256 MiB copy and of the RS(6,3) encode, for counter runs; "
                         "batched: configs 4 and 5 only; batched-kernels: the same without "
                         "the checkpoint staging and snapshot (for kernel-trace profiles); "
                         "batched-pmc: the copy plus 3 launches of each batched kernel, for "
                         "counter runs; train: a training "
                         "loop with synchronous and with snapshot checkpoint saves; "
                         "small-shards: RS(6,3) over 1 and 4 MiB shards, eager and planned; "
                         "layout: RS(6,3) over config 2's bytes as six shards, cut into "
                         "units, and stripe-contiguous")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the erasure-coding path has no multi-GPU "
              f"component in this build (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from megatron_lm_amd import synth
    pkg._lib.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.mode == "pmc":
        return pmc_launches(pkg, dev)
    if args.mode in ("batched", "batched-kernels"):
        print(json.dumps({"mode": args.mode,
                          **batched_configs(pkg, synth, dev, args.seed, GemmLoad(dev),
                                            with_checkpoint=args.mode == "batched")}),
              flush=True)
        return 0
    if args.mode == "batched-pmc":
        return batched_pmc_launches(pkg, synth, dev, args.seed)
    if args.mode == "small-shards":
        print(json.dumps({"mode": args.mode, **small_shards(pkg, dev)}), flush=True)
        return 0
    if args.mode == "layout":
        data = [torch.from_numpy(h).to(dev) for h in synth.rs_shards(args.seed, 256 * MiB, 6)]
        print(json.dumps({"mode": args.mode, **stripe_layouts(pkg, dev, data)}), flush=True)
        return 0
    if args.mode == "train":
        print(json.dumps({"mode": "train", **training_with_checkpoints(pkg, dev)}), flush=True)
        return 0

    # ---- config 2: RS(6,3), 6 x 256 MiB fp32 optimizer state -------------
    k, m, shard = 6, 3, 256 * MiB
    log("generating RS(6,3) shards (numpy, seeded)")
    host = synth.rs_shards(args.seed, shard, k)
    data = [torch.from_numpy(h).to(dev) for h in host]
    parity = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in range(m)]
    coeff = pkg.cauchy_matrix(k, m)
    data_bytes = k * shard
    traffic = (k + m) * shard

    encode = lambda: pkg.matvec(coeff, data, out=parity)
    settle_ms, settle_n = settle(encode, args.settle_ms * 1e-3)
    log(f"RS(6,3) encode: settled {settle_ms:.0f} ms ({settle_n} launches), then "
        f"{args.warmup} warmup + {args.steps} timed steps")
    wall_ms, ev_ms = timed(encode, args.steps, args.warmup)
    enc_gbs = data_bytes / (wall_ms * 1e-3) / 1e9
    enc_traffic_gbs = traffic / (ev_ms * 1e-3) / 1e9
    spread = launch_spread(encode, args.steps)
    log(f"encode {enc_gbs:.1f} GB/s data, kernel {ev_ms*1e3:.1f} us, "
        f"{enc_traffic_gbs:.0f} GB/s HBM traffic; per launch median "
        f"{spread['median']*1e3:.1f} us, min {spread['min']*1e3:.1f}, "
        f"max {spread['max']*1e3:.1f}")

    if args.mode == "headline":
        print(json.dumps({"mode": "headline", "encode_GBps": round(enc_gbs, 2),
                          "kernel_us": round(ev_ms * 1e3, 2),
                          "kernel_us_median": round(spread["median"] * 1e3, 2),
                          "settle_ms": round(settle_ms, 1),
                          "traffic_GBps": round(enc_traffic_gbs, 1)}), flush=True)
        return 0

    # ---- config 3: decode 3 seeded erasures of the same codeword ----------
    lost = synth.erasures(args.seed, k + m, m)
    codeword = data + parity
    surv, rows = pkg.decode_matrix(coeff, lost)
    survivors = [codeword[s] for s in surv]
    recovered = [torch.empty(shard, dtype=torch.uint8, device=dev) for _ in lost]
    dwall, dev_ms = steady(lambda: pkg.matvec(rows, survivors, out=recovered, what="ec_rs_decode"),
                           max(1, args.steps // 2), max(1, args.warmup // 2))
    torch.cuda.synchronize()
    if not all(torch.equal(r, codeword[g]) for r, g in zip(recovered, lost)):
        raise AssertionError("decode did not reproduce the lost shards")
    dec_gbs = data_bytes / (dwall * 1e-3) / 1e9
    log(f"decode lost={lost}: {dec_gbs:.1f} GB/s data")
    if args.mode == "decode":
        print(json.dumps({"mode": "decode", "lost": lost, "decode_GBps": round(dec_gbs, 2),
                          "kernel_us": round(dev_ms * 1e3, 2),
                          "traffic_GBps": round(traffic / (dev_ms * 1e-3) / 1e9, 1)}), flush=True)
        return 0

    # ---- config 1: XOR, 4 x 64 MiB bf16 ----------------------------------
    xh = synth.xor_shards(args.seed, 64 * MiB, 4)
    xd = [torch.from_numpy(h).to(dev) for h in xh]
    xp = torch.empty(64 * MiB, dtype=torch.uint8, device=dev)
    xwall, xev = steady(lambda: pkg.xor_encode(xd, out=xp), args.steps, args.warmup)
    # Product-only check: XOR of the parity with the first k-1 shards gives back the last.
    back = pkg.xor_encode(xd[:3] + [xp])
    torch.cuda.synchronize()
    if not torch.equal(back, xd[3]):
        raise AssertionError("XOR parity does not reproduce the shards")
    xor_gbs = 4 * 64 * MiB / (xwall * 1e-3) / 1e9
    log(f"XOR(4) {xor_gbs:.1f} GB/s data")
    if args.mode == "flat-kernels":
        del xd, xp, back
        src = torch.empty(k * shard, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        _, cev = timed(lambda: pkg.xor_encode([src], out=dst), 50, 10)
        print(json.dumps({"mode": "flat-kernels", "encode_GBps": round(enc_gbs, 2),
                          "encode_kernel_us": round(ev_ms * 1e3, 2),
                          "decode_GBps": round(dec_gbs, 2), "decode_kernel_us": round(dev_ms * 1e3, 2),
                          "xor_GBps": round(xor_gbs, 2), "xor_kernel_us": round(xev * 1e3, 2),
                          "copy_kernel_us": round(cev * 1e3, 2),
                          "copy_GBps": round(2 * src.numel() / (cev * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    small = small_shards(pkg, dev)
    layouts = stripe_layouts(pkg, dev, data)

    gemm = GemmLoad(dev)
    batched = {} if args.no_batched else batched_configs(
        pkg, synth, dev, args.seed, gemm, 0.0 if args.no_cpu_baseline else args.cpu_seconds / 5)
    batched_cpu = batched.pop("cpu", {})
    log("encode on a side stream vs bf16 GEMMs")
    over = overlap_with_training(pkg, dev, data, parity, coeff, gemm)
    del gemm
    torch.cuda.empty_cache()
    log("training loop with checkpoint saves (its own process)")
    over.update(training_in_child())

    # ---- practical ceiling: the engine's streaming copy (XOR of one shard,
    # same loads/stores as the kernels) and torch's device-to-device copy ---
    src = torch.empty(k * shard, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    cwall, cev = timed(lambda: pkg.xor_encode([src], out=dst), 50, 10)
    copy_gbs = 2 * src.numel() / (cev * 1e-3) / 1e9
    twall, tev = timed(lambda: dst.copy_(src), 20, 3)
    torch_copy_gbs = 2 * src.numel() / (tev * 1e-3) / 1e9
    del src, dst
    log(f"streaming copy {copy_gbs:.0f} GB/s, torch D2D copy {torch_copy_gbs:.0f} GB/s (read+write)")
    skel = skeleton_ceilings(pkg, dev, shard, enc_traffic_gbs)
    log(f"memory skeleton: {skel}")

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline")
        cpu = cpu_baseline(host, k, m, args.cpu_seconds, parity, xh, xp, lost, batched_cpu)
        cpu["configs"]["xor_4x64MiB"]["gpu_GBps"] = round(xor_gbs, 1)
        cpu["configs"]["rs63_decode_3_erasures"]["gpu_GBps"] = round(dec_gbs, 1)
        log(f"CPU {cpu['value']} GB/s on {cpu['cores']} cores, {cpu['one_core_GBps']} GB/s on 1")

    result = {
        "metric": "RS(6,3) encode GB/s (data bytes) on 1 MI355X + % HBM roofline; decode GB/s",
        "value": round(enc_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded numpy: fp32 master N(0,0.02) x2, exp_avg N(0,1e-3) x2, "
                "exp_avg_sq |N(0,1e-6)| x2)",
        "config": {"workload": "RS(6,3) encode over GF(2^8)/0x11D, Cauchy generator, "
                               "6 x 256 MiB data shards -> 3 x 256 MiB parity",
                   "k": k, "m": m, "shard_bytes": shard, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(enc_traffic_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(enc_traffic_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(k, m, shard),
                     "kernel": "rs_kernel<6,3>",
                     "algorithmic_bytes_per_launch": traffic,
                     "kernel_us": round(ev_ms * 1e3, 2),
                     "settle_ms": round(settle_ms, 1),
                     "settle_launches": settle_n,
                     "launch_us_median": round(spread["median"] * 1e3, 2),
                     "launch_us_min": round(spread["min"] * 1e3, 2),
                     "launch_us_max": round(spread["max"] * 1e3, 2),
                     "launch_us_mean_per_launch_events": round(spread["mean"] * 1e3, 2)},
        "cpu_baseline": cpu,
        "also": {
            "decode_GBps": round(dec_gbs, 2), "decode_lost": lost,
            "decode_kernel_us": round(dev_ms * 1e3, 2),
            "xor_4x64MiB_GBps": round(xor_gbs, 2), "xor_kernel_us": round(xev * 1e3, 2),
            **small,
            "stripe_layouts": layouts,
            **batched,
            **over,
            "copy_ceiling_GBps": round(copy_gbs, 1),
            "torch_d2d_copy_GBps": round(torch_copy_gbs, 1),
            "encode_frac_of_copy_ceiling": round(enc_traffic_gbs / copy_gbs, 4),
            **skel,
        },
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
