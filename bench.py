"""Benchmark of the weight-streaming path on one MI355X.

Headline workload (``value``): the Llama-style 32-layer decoder at 7B shape
(hidden 4096, 32 heads, SwiGLU 11008, vocab 32000; bf16 weights N(0, 0.02)
from seed 0) under an 8 GB GPU weight budget. A 512-token prompt is
prefilled, then ``--warmup`` greedy batch-1 decode tokens run untimed and
``--steps`` decode tokens are timed: a step is one decode token, a full pass
over the model that streams every layer outside the budget from pinned host
memory. ``value`` = streamed bytes per token x tokens / wall time (effective
streamed-weight GB/s), beside the measured host-link peak (best of 20
512 MiB copies) and the token rate. The weights are host-resident by
definition of the workload, so ``value`` is host-link inclusive.

Beside it, on the same line: the scatter microbenchmark (2000 bf16 tensors
log-uniform in [4 KiB, 64 MiB], 512 MiB pinned chunks, one scatter launch per
chunk) with the scatter kernel's HBM roofline (``roofline``) and its
rocprofv3 traffic; the 8-layer MLP stack; the Wan-style DiT step against a
measured resident step; the fp8 decode GEMM on one 70B layer; the 80-layer
70B fp8 batch-8 decode. CPU baselines are timed on the host cores.

Only one GPU is used: ``--gpus`` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

MiB = 1 << 20
HBM_PEAK_GBPS = 8000.0
PCIE_GEN5_X16_GBPS = 63.0  # 32 GT/s x 16 lanes x 128/130 / 8
# Offload units one level below a decoder layer: attention, gate, up and down (the norms stay resident).
FINER_UNITS = ("layers.*.attn", "layers.*.gate", "layers.*.up", "layers.*.down")


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measure_link_peak(repeats: int = 20) -> dict:
    from flextensor_amd.link_model import time_h2d

    out = {}
    for engine in ("sdma", "kernel"):
        t = time_h2d(512 * MiB, engine, repeats=repeats, warmup=2)
        out[engine] = 512 * MiB / (min(t) * 1e-3) / 1e9
    return out


def bench_scatter(steps: int, warmup: int, chunk_mib: int, n_tensors: int, copy_engine: str,
                  verify: bool = True) -> dict:
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd import workloads as W
    from flextensor_amd.hip import HostArena
    from flextensor_amd.scatter import ChunkedUploader, plan_chunks

    dev = torch.device("cuda", 0)
    sizes = W.scatter_sizes(n_tensors, 4096, 64 * MiB, seed=1)
    chunks = plan_chunks(sizes, chunk_mib * MiB)
    payload = sum(sizes)
    _log(f"scatter set: {n_tensors} tensors, {payload / 1e9:.2f} GB in {len(chunks)} chunks of <= {chunk_mib} MiB")
    gen = torch.Generator(device=dev).manual_seed(1)
    for ch in chunks:
        ch.host = HostArena(ch.nbytes).tensor
        ch.host.copy_(torch.randint(0, 256, (ch.nbytes,), dtype=torch.uint8, device=dev, generator=gen))
    dests = [torch.empty(W.scatter_shape(n, i), dtype=torch.bfloat16, device=dev) for i, n in enumerate(sizes)]
    up = ChunkedUploader(chunks, dests, dev, n_slots=2, copy_mode=nat.COPY_MODES[copy_engine])
    for _ in range(warmup):
        up.upload()
    torch.cuda.synchronize()
    timing: list = []
    t0 = time.perf_counter()
    for _ in range(steps):
        up.upload(timing)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    copy_ms = sum(e[0].elapsed_time(e[1]) for e in timing)
    scat_ms = [e[2].elapsed_time(e[3]) for e in timing]
    chunk_bytes = [ch.nbytes for ch in chunks] * steps
    scat_payload = [sum(p.nbytes for p in ch.pieces) for ch in chunks] * steps
    # verification through torch's own copy path, independent of the engine under test
    bad = 0
    for ch in chunks if verify else []:
        ref = ch.host.to(dev)
        for p in ch.pieces:
            if p.nbytes:
                got = dests[p.index].view(-1).view(torch.uint8)[p.tensor_off: p.tensor_off + p.nbytes]
                bad += int(not torch.equal(got, ref[p.chunk_off: p.chunk_off + p.nbytes]))
        del ref
    avg_scatter_ms = sum(scat_ms) / len(scat_ms)
    res = {
        "ms_per_step": wall * 1e3,
        "payload_bytes": payload,
        "n_chunks": len(chunks),
        "effective_GBps": payload / wall / 1e9,
        "link_GBps": sum(chunk_bytes) / (copy_ms * 1e-3) / 1e9,
        "scatter_avg_ms": avg_scatter_ms,
        "scatter_hbm_GBps": 2 * sum(scat_payload) / (sum(scat_ms) * 1e-3) / 1e9,
        "scatter_bytes_per_launch": 2 * payload / len(chunks),
        "mismatched_tensors": bad,
        "chunks": chunks,
    }
    up.close()
    return res


def device_copy_probe(nbytes: int, reps: int = 10) -> dict:
    """The runtime's own device-to-device copy (``Tensor.copy_`` -> ``hipMemcpyAsync``) of ``nbytes``: the plain
    copy rate the scatter kernel (which reads and writes the same bytes) is compared with. Best of ``reps``,
    HIP events on torch's stream; GB/s count bytes read plus bytes written."""
    import torch

    dev = torch.device("cuda", 0)
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        b.synchronize()
        best = min(best, a.elapsed_time(b))
    ok = bool(torch.equal(dst, src))
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "GBps": round(2 * nbytes / best / 1e6, 1), "ms": round(best, 4), "bit_exact": ok}


def cpu_baseline_scatter(chunks, sample_chunks: int = 4, reps: int = 3, threads: int = 16) -> dict:
    """The oracle's byte scatter (memcpy per descriptor) over the first chunks of the same workload, on
    ``threads`` host threads: each thread scatters a contiguous share of each chunk's descriptors (the
    oracle's C call releases the interpreter lock)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle import native as onat

    sample = chunks[:sample_chunks]
    extent: dict[int, int] = {}
    for ch in sample:
        for p in ch.pieces:
            extent[p.index] = max(extent.get(p.index, 1), p.tensor_off + p.nbytes)
    dsts = {i: np.empty(n, np.uint8) for i, n in extent.items()}
    nbytes = sum(p.nbytes for ch in sample for p in ch.pieces)
    jobs = []
    for ch in sample:
        host = ch.host.numpy()
        pieces = sorted(ch.pieces, key=lambda q: q.chunk_off)
        share = max(1, -(-sum(q.nbytes for q in pieces) // threads))
        part, size = [], 0
        for q in pieces:  # contiguous shares of about equal bytes
            part.append(q)
            size += q.nbytes
            if size >= share:
                jobs.append((host, part))
                part, size = [], 0
        if part:
            jobs.append((host, part))

    def run(job):
        host, part = job
        onat.scatter(host, [(q.chunk_off, q.nbytes) for q in part], [dsts[q.index][q.tensor_off:] for q in part])

    best = float("inf")
    with ThreadPoolExecutor(threads) as pool:
        for _ in range(reps):
            t0 = time.perf_counter()
            list(pool.map(run, jobs))
            best = min(best, time.perf_counter() - t0)
    return {"value": nbytes / best / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle scatter (memcpy per descriptor) of the first {len(sample)} chunks, {nbytes / 1e9:.2f} GB, "
                      f"on {threads} threads, best of {reps}"}


def ring_copy_stats(mgr, step, tokens: int) -> dict | None:
    """Every ring copy of ``tokens`` more streamed passes, timed one by one.

    The offload timing collector (HIP events on the transfer stream around
    each copy, offload_timing.py:31-44) is switched on for these passes only,
    after the timed ones, so its per-pass synchronize cannot slow them.
    ``step()`` runs one pass. Returns launches, mean microseconds and GB/s per
    copy size, and the size that moves the most bytes.
    """
    import torch

    from flextensor_amd.timing import OffloadTimingCollector

    if mgr.controller is None:  # everything resident: no ring copies
        return None
    collector = OffloadTimingCollector(list(mgr.order))
    loader = mgr.loader
    kept, loader.offload_timing_collector = loader.offload_timing_collector, collector
    try:
        for _ in range(tokens):
            step()
        torch.cuda.synchronize()
        report = collector.report()
    finally:
        loader.offload_timing_collector = kept
    by_size: dict[int, list[float]] = {}
    link: dict[int, list[int]] = {}  # bytes each launch read over the link (less than n for an encoded block)
    ctl = mgr.controller
    for snap in report.passes:
        for rec in snap.per_trap:
            if rec.transfer_ms > 0:
                n = ctl.transfer_bytes(rec.label)
                by_size.setdefault(n, []).append(rec.transfer_ms)
                link.setdefault(n, []).append(ctl.link_bytes(rec.label) if hasattr(ctl, "link_bytes") else n)
    sizes = {n: {"launches": len(ms), "mean_us": round(1e3 * sum(ms) / len(ms), 1),
                 "GBps": round(n * len(ms) / sum(ms) / 1e6, 3)} for n, ms in sorted(by_size.items())}
    for n, v in sizes.items():
        if sum(link[n]) != n * len(link[n]):
            v["link_bytes_mean"] = round(sum(link[n]) / len(link[n]))
            v["link_GBps"] = round(sum(link[n]) / sum(by_size[n]) / 1e6, 3)
    top = max(by_size, key=lambda n: n * len(by_size[n]))
    return {"passes": report.num_passes, "by_size": {str(n): v for n, v in sizes.items()}, "dominant_bytes": top,
            "dominant": sizes[top]}


def bench_llama7b(budget_gb: float, prefill: int, steps: int, warmup: int, copy_engine: str,
                  include_patterns: tuple[str, ...] = ("layers.*",), ring_tokens: int = 4,
                  ring_order: str = "auto", encode: bool = False, encode_resident: bool = False,
                  link_benchmark: bool = True) -> dict:
    """Prefill, then ``warmup`` untimed and ``steps`` timed greedy decode tokens of the 7B-shape decoder
    streaming under ``budget_gb`` (a step is one decode token). ``include_patterns`` choose the offload
    units: whole decoder layers by default. The prefill's last-position logits and every decoded token are
    returned under ``_check`` so that runs with other units can be compared bitwise. After the timed
    tokens, ``ring_tokens`` more decode tokens time every ring copy on its own (:func:`ring_copy_stats`).
    ``ring_order`` "reference" or "link-bound" overrides how the ring's copies are waited for
    (:func:`_set_ring_order`). ``encode`` streams the blocks exponent-coded
    (``OffloadConfig.encode_streamed_blocks``); ``encode_resident`` keeps resident layers exponent-coded
    in HBM when they do not fit raw (``OffloadConfig.encode_resident_blocks``), so fewer layers stream.
    ``link_benchmark`` False skips the host-link measurement (``OffloadConfig.link_benchmark``): no pass
    regime is measured, so every streamed block that shrinks is encoded. Under a kernel tracer the
    profiled compute of the pass is inflated and the measured regime would differ from an untraced run;
    with ``ring_order="link-bound"`` this reproduces the untraced link-bound configuration."""
    import torch

    from flextensor_amd import hip
    from flextensor_amd import workloads as W
    from flextensor_amd.config import OffloadConfig
    from flextensor_amd.manager import OffloadManager

    dev = torch.device("cuda", 0)
    t0 = time.perf_counter()
    model = W.build_llama(W.LLAMA_7B, seed=0, init_device="cuda")
    _log(f"llama7b: built in {time.perf_counter() - t0:.1f} s")
    mgr = OffloadManager("bench-llama")
    cfg = OffloadConfig(include_patterns=list(include_patterns), num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=int(budget_gb * 1e9), copy_engine=copy_engine,
                        encode_streamed_blocks=encode, encode_resident_blocks=encode_resident,
                        link_benchmark=link_benchmark)
    mgr.offload(model, cfg)
    prompt = W.prompt_tokens(1, prefill, W.LLAMA_7B.vocab, seed=0).to(dev)
    total = prefill + warmup + steps + ring_tokens + 2
    model.init_cache(1, total, dev)
    with torch.no_grad():
        model(prompt[:, :16], 0)  # discovery
        model(prompt[:, :16], 0)  # profiling -> plan and loader are built here
    _log(f"llama7b: streaming set up ({mgr.build_seconds:.1f} s to pack, measure the link and build)")
    _set_ring_order(mgr, ring_order)
    plan = mgr.plan
    streamed_bytes = sum(mgr._unit(x).nbytes for x in plan.streamed)
    ctl = mgr.controller
    hbm = getattr(ctl, "hbm_encoded", {}) or {}
    link_bytes = sum(ctl.link_bytes(x) for x in ctl.block_map_cpu if x not in hbm) if ctl is not None else 0
    encoded = len(getattr(ctl, "encoded", {}) or {})
    hbm_bytes = sum(b.capacity for b in hbm.values())
    with torch.no_grad():
        model.init_cache(1, total, dev)
        W.generate(model, prompt, 2)  # warm-up pass
        model.init_cache(1, total, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = model(prompt, 0)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        last_logits = logits[:, -1].float().cpu()
        tok = logits.argmax(-1)
        toks = [tok]
        pos = prefill
        for _ in range(warmup):
            tok = model(tok, pos).argmax(-1)
            toks.append(tok)
            pos += 1
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = model(tok, pos).argmax(-1)
            toks.append(tok)
            pos += 1
        torch.cuda.synchronize()
        t_decode = time.perf_counter() - t0
        state = {"tok": tok, "pos": pos}

        def one_token():
            state["tok"] = model(state["tok"], state["pos"]).argmax(-1)
            state["pos"] += 1

        ring = ring_copy_stats(mgr, one_token, ring_tokens) if ring_tokens else None
    usage = mgr.get_gpu_memory_usage()
    link = mgr.link.to_dict() if mgr.link is not None else None
    out = {
        "prefill_tokens": prefill,
        "decode_steps": steps,
        "decode_warmup": warmup,
        "prefill_tok_s": prefill / t_prefill,
        "decode_tok_s": steps / t_decode,
        "ms_per_token": 1e3 * t_decode / steps,
        "streamed_bytes_per_token": streamed_bytes,
        "decode_effective_GBps": streamed_bytes * steps / t_decode / 1e9,
        "link_bytes_per_token": link_bytes,
        "decode_link_GBps": link_bytes * steps / t_decode / 1e9,
        "encoded_blocks": encoded,
        "hbm_encoded_layers": len(hbm),
        "hbm_encoded_bytes": hbm_bytes,
        "hbm_encoded_ratio": round(hbm_bytes / sum(b.raw_bytes for b in hbm.values()), 4) if hbm else None,
        "streamed_layers": len(plan.streamed),
        "resident_layers": len(plan.resident),
        "gpu_weight_bytes": usage.total_bytes,
        "budget_bytes": int(budget_gb * 1e9),
        "copy_policy": None if link is None else {k: link[k] for k in ("kernel_max_bytes", "split_min_bytes",
                                                                       "n_copy_streams", "kernel_grid",
                                                                       "link_bound", "pass_compute_ms",
                                                                       "pass_transfer_ms")},
        "copy_policy_source": None if mgr.link is None else mgr.link.source,
        "transfer_stream": hip.transfer_stream_probe(dev),
        "ring_copies": ring,
        "ring_copy_engine": _ring_engine(mgr),
        "ring_order": _ring_order(mgr),
        "_check": {"last_logits": last_logits, "tokens": torch.cat(toks, -1).cpu()},
    }
    mgr.release(preserve_model=False)
    return out


def _ring_roofline(run: dict, measured_peak: float) -> dict | None:
    """The host-link roofline of a decode's dominant kernel, its ring copy: bytes per launch over the mean
    launch time, against PCIe Gen5 x16 and against the measured link peak (512 MiB, best of 20)."""
    ring = run.get("ring_copies")
    if not ring:
        return None
    d = ring["dominant"]
    link = d.get("link_GBps", d["GBps"])  # an encoded block moves fewer bytes over the link than it writes
    out = {"kernel": run["ring_copy_engine"], "bound": "host link (PCIe Gen5 x16)", "achieved": link,
           "peak": PCIE_GEN5_X16_GBPS, "unit": "GB/s", "frac": round(link / PCIE_GEN5_X16_GBPS, 4),
           "frac_of_measured_peak": round(link / measured_peak, 4), "traffic": None,
           "bytes_per_launch": ring["dominant_bytes"], "avg_launch_us": d["mean_us"], "launches": d["launches"],
           "timing": f"HIP events on the transfer stream around each ring copy, over {ring['passes']} decode "
                     "tokens after the timed ones",
           "by_size": ring["by_size"]}
    if "link_GBps" in d:
        out["link_bytes_per_launch"] = d["link_bytes_mean"]
        out["raw_bytes_written_GBps"] = d["GBps"]
    return out


def expcode_sweep(grids=(8, 16, 32, 64, 128), reps: int = 6, hbm_grids=(0, 256, 512, 1024, 2048, 4096)) -> dict:
    """One 7B layer's block (404,766,720 bytes of N(0, 0.02) bf16) encoded, then decoded into the device by
    ``expcode_decode_kernel`` at each grid, against the raw block's zero-copy copy and SDMA copy; then the
    same decode from a device-memory copy of the encoded block at ``hbm_grids`` (0: the library's eight per CU)
    against a device-to-device copy of the raw block. Best of ``reps`` HIP-event timings per case; every
    decode is checked bit for bit."""
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd import expcode
    from flextensor_amd.hip import HostArena, copy_h2d

    from flextensor_amd import workloads as W

    n = W.LLAMA_7B.layer_bytes()
    g = torch.Generator().manual_seed(0)
    arena = HostArena(n)
    arena.tensor[:n].copy_((torch.randn(n // 2, generator=g) * 0.02).to(torch.bfloat16).view(torch.uint8))
    raw = arena.tensor[:n]
    t0 = time.perf_counter()
    block = expcode.encode(raw)
    encode_s = time.perf_counter() - t0
    dst = torch.empty(n, dtype=torch.uint8, device="cuda")
    ref = raw.to("cuda")

    def best(fn) -> float:
        ms = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            fn()
            b.record()
            b.synchronize()
            ms.append(a.elapsed_time(b))
        return min(ms)

    out = {"raw_bytes": n, "encoded_bytes": block.nbytes, "ratio": round(block.ratio, 4),
           "encode_s": round(encode_s, 3), "decode": {}}
    for grid in grids:
        pol = nat.copy_policy(0, 2**63 - 1, 1, grid)
        dst.zero_()
        ms = best(lambda: expcode.decode_h2d(dst, block, policy=pol))
        out["decode"][str(grid)] = {"ms": round(ms, 3), "raw_GBps": round(n / ms / 1e6, 2),
                                    "link_GBps": round(block.nbytes / ms / 1e6, 2),
                                    "bit_exact": bool(torch.equal(dst, ref))}
    # the dense format (version 2) over the link
    dense_link = expcode.encode(raw, dense=True)
    out["dense_link"] = {"encoded_bytes": dense_link.nbytes, "ratio": round(dense_link.ratio, 4), "decode": {}}
    for grid in grids:
        pol = nat.copy_policy(0, 2**63 - 1, 1, grid)
        dst.zero_()
        ms = best(lambda: expcode.decode_h2d(dst, dense_link, policy=pol))
        out["dense_link"]["decode"][str(grid)] = {"ms": round(ms, 3), "raw_GBps": round(n / ms / 1e6, 2),
                                                  "link_GBps": round(dense_link.nbytes / ms / 1e6, 2),
                                                  "bit_exact": bool(torch.equal(dst, ref))}
    del dense_link
    pol = nat.copy_policy(1 << 40, 2**63 - 1, 1, 8)
    ms = best(lambda: copy_h2d(dst, raw, nat.COPY_KERNEL, policy=pol))
    out["zero_copy_raw_8_workgroups"] = {"ms": round(ms, 3), "GBps": round(n / ms / 1e6, 2)}
    ms = best(lambda: copy_h2d(dst, raw, nat.COPY_SDMA))
    out["sdma_raw"] = {"ms": round(ms, 3), "GBps": round(n / ms / 1e6, 2)}
    # The same block kept in device memory (a unit resident in HBM in encoded form): the decode reads
    # the encoded bytes and writes the raw ones, both in HBM. Grid 0 is the library's default.
    src = block.tensor.to("cuda")
    moved = block.nbytes + n
    out["decode_from_hbm"] = {}
    for grid in hbm_grids:
        dst.zero_()
        ms = best(lambda: expcode.decode_d2d(dst, src, n, grid=grid))
        out["decode_from_hbm"][str(grid)] = {"us": round(1e3 * ms, 1), "hbm_GBps": round(moved / ms / 1e6, 1),
                                             "frac_of_8TBps": round(moved / ms / 1e6 / 8000, 4),
                                             "bit_exact": bool(torch.equal(dst, ref))}
    ms = best(lambda: dst.copy_(ref))
    out["device_copy_raw"] = {"us": round(1e3 * ms, 1), "hbm_GBps": round(2 * n / ms / 1e6, 1)}
    # The dense format (version 2) that units kept in HBM use
    t0 = time.perf_counter()
    dense = expcode.DeviceEncodedBlock.from_raw(raw, expcode.encoded_size(raw, dense=True), "cuda", dense=True)
    dense_s = time.perf_counter() - t0
    moved = dense.nbytes + n
    out["dense"] = {"encoded_bytes": dense.nbytes, "ratio": round(dense.ratio, 4),
                    "encode_and_upload_s": round(dense_s, 3), "decode_from_hbm": {}}
    for grid in hbm_grids:
        dst.zero_()
        ms = best(lambda: expcode.decode_d2d(dst, dense.dev, n, grid=grid, dense=True))
        out["dense"]["decode_from_hbm"][str(grid)] = {
            "us": round(1e3 * ms, 1), "hbm_GBps": round(moved / ms / 1e6, 1),
            "frac_of_8TBps": round(moved / ms / 1e6 / 8000, 4), "bit_exact": bool(torch.equal(dst, ref))}
    return out


def _encoded_summary(enc: dict, measured_peak: float, raw_tok_s: float | None) -> dict:
    """The 7B decode with exponent-coded blocks: weight bytes per token against the bytes that crossed
    the link, the effective weight rate and the link's own rate."""
    return {
        "encoded_blocks": enc["encoded_blocks"], "streamed_layers": enc["streamed_layers"],
        "resident_layers": enc["resident_layers"], "hbm_encoded_layers": enc["hbm_encoded_layers"],
        "hbm_encoded_ratio": enc["hbm_encoded_ratio"], "gpu_weight_bytes": enc["gpu_weight_bytes"],
        "streamed_bytes_per_token": enc["streamed_bytes_per_token"],
        "link_bytes_per_token": enc["link_bytes_per_token"],
        "link_bytes_ratio": round(enc["link_bytes_per_token"] / enc["streamed_bytes_per_token"], 4),
        "tok_s": round(enc["decode_tok_s"], 3), "ms_per_token": round(enc["ms_per_token"], 3),
        "decode_effective_GBps": round(enc["decode_effective_GBps"], 3),
        "decode_link_GBps": round(enc["decode_link_GBps"], 3),
        "link_pct_of_measured_peak": round(100 * enc["decode_link_GBps"] / measured_peak, 2),
        "speedup_vs_raw_blocks": None if raw_tok_s is None else round(enc["decode_tok_s"] / raw_tok_s, 4),
        "prefill_tok_s": round(enc["prefill_tok_s"], 1),
        "ring_order": enc["ring_order"],
        "regime": None if enc["copy_policy"] is None else {k: enc["copy_policy"][k] for k in
                                                           ("link_bound", "pass_compute_ms", "pass_transfer_ms")},
        "ring_copies": _ring_roofline(enc, measured_peak),
    }


def _set_ring_order(mgr, how: str) -> None:
    """Override the manager's choice of ring order: "reference" (the reference's order: the compute stream
    waits on each copy's ready event) or "link-bound" (the reordered loader blocks the host on it with the
    next copy queued; the default loader releases a unit's slots before its wait); "auto" keeps the
    manager's choice (link-bound for a link-bound pass)."""
    if how != "auto" and hasattr(mgr.loader, "link_bound"):
        mgr.loader.link_bound = how == "link-bound"


def _ring_order(mgr) -> str:
    return "link-bound" if getattr(mgr.loader, "link_bound", False) else "reference"


def _ring_engine(mgr) -> str:
    """Which engine the manager's ring copies run on: its copy mode and the policy its controller carries."""
    from flextensor_amd import _native as nat

    ctl = mgr.controller
    if getattr(ctl, "encoded", None):
        dense = any(getattr(b, "dense", False) for b in ctl.encoded.values())
        return f"{'expcode_dense_link_decode_kernel' if dense else 'expcode_decode_kernel'} (16 workgroups)"
    mode, policy = ctl.copy_mode, ctl.copy_policy
    if mode == nat.COPY_AUTO:
        if policy is None:
            policy = nat.copy_policy(*nat.get_copy_policy())
        biggest = max(ctl.transfer_bytes(x) for x in ctl.block_map_cpu)
        mode = nat.COPY_KERNEL if biggest <= policy.kernel_max_bytes else nat.COPY_SDMA
    if mode == nat.COPY_KERNEL:
        grid = (policy.kernel_grid if policy is not None else nat.get_copy_policy()[3]) or 64
        return f"zero_copy_kernel ({grid} workgroups)"
    return "SDMA (hipMemcpyAsync)" if mode == nat.COPY_SDMA else "staged"


def bench_mlp(steps: int, copy_engine: str, ring_order: str = "auto", encode: bool = False) -> dict:
    """The 8-layer 4096->11008->4096 MLP stack, every layer streamed through a 2-slot ring.

    Times ``steps`` eager streamed forwards, then the same forward captured in
    a HIP graph and replayed ``steps`` times; both outputs are checked bitwise
    against the all-resident forward. The CPU baseline is the same forward in
    PyTorch on the host cores. ``encode`` streams the blocks exponent-coded
    (``OffloadConfig.encode_streamed_blocks``; no CPU baseline then).
    """
    import torch

    from flextensor_amd import workloads as W
    from flextensor_amd.config import OffloadConfig
    from flextensor_amd.manager import OffloadManager

    dev = torch.device("cuda", 0)
    model = W.build_mlp_stack(8, 4096, 11008, seed=0)
    x = W.mlp_input(16, 4096, seed=0).to(dev)
    resident = W.build_mlp_stack(8, 4096, 11008, seed=0).to(dev)
    with torch.no_grad():
        want = resident(x)
    del resident
    streamed_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    mgr = OffloadManager("bench-mlp")
    mgr.offload(model, OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                                     profiling_iters=1, copy_engine=copy_engine, encode_streamed_blocks=encode))
    with torch.no_grad():
        for _ in range(2):  # discovery, then profiling: the plan and the loader are built at its end
            out = model(x)
        ctl = mgr.controller
        link_bytes = sum(ctl.link_bytes(label) for label in ctl.block_map_cpu)
        encoded = len(ctl.encoded)
        _set_ring_order(mgr, ring_order)
        order = _ring_order(mgr)
        for _ in range(2):  # two streamed warm-up passes
            out = model(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = model(x)
        torch.cuda.synchronize()
        t_eager = (time.perf_counter() - t0) / steps
    eager_ok = bool(torch.equal(out, want))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        model(x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s), torch.no_grad():
        static_out = model(x)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    t_graph = (time.perf_counter() - t0) / steps
    graph_ok = bool(torch.equal(static_out, want))
    del g, static_out
    mgr.release(preserve_model=True)
    out = {
        "streamed_bytes_per_forward": streamed_bytes,
        "link_bytes_per_forward": link_bytes,
        "encoded_blocks": encoded,
        "eager_ms_per_forward": 1e3 * t_eager,
        "eager_effective_GBps": streamed_bytes / t_eager / 1e9,
        "eager_link_GBps": link_bytes / t_eager / 1e9,
        "graph_ms_per_forward": 1e3 * t_graph,
        "graph_effective_GBps": streamed_bytes / t_graph / 1e9,
        "graph_link_GBps": link_bytes / t_graph / 1e9,
        "ring_order": order,
        "bitwise_equal_to_resident": eager_ok and graph_ok,
    }
    if encode:
        return out
    # CPU baseline: the same forward in PyTorch on the host cores
    xc = x.cpu()
    with torch.no_grad():
        for _ in range(2):
            model(xc)
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            model(xc)
            ts.append(time.perf_counter() - t0)
    t_cpu = sorted(ts)[len(ts) // 2]
    out["cpu_baseline"] = {"value": 1e3 * t_cpu, "unit": "ms per forward", "cores": torch.get_num_threads(),
                           "kind": "port", "sample": "the full 8-layer bf16 forward on the host cores, median of 5"}
    return out


def cpu_llama_decode_baseline(layers: int = 2, tokens: int = 4, context: int = 512) -> dict:
    """Batch-1 decode of ``layers`` 7B-shape decoder layers in PyTorch on the host cores, scaled to 32 layers."""
    import torch

    from flextensor_amd import workloads as W

    s = W.LlamaShape(n_layers=layers, vocab=256)
    model = W.build_llama(s, seed=0)
    model.init_cache(1, context + tokens + 2, torch.device("cpu"))
    x = torch.randn(1, 1, s.hidden, dtype=torch.bfloat16)
    with torch.no_grad():
        for i in range(2):
            for layer_i, layer in enumerate(model.layers):
                layer(x, context + i, model.rope_cos, model.rope_sin, model.cache_k[layer_i], model.cache_v[layer_i])
        t0 = time.perf_counter()
        for i in range(tokens):
            for layer_i, layer in enumerate(model.layers):
                layer(x, context + 2 + i, model.rope_cos, model.rope_sin, model.cache_k[layer_i],
                      model.cache_v[layer_i])
        per_layer = (time.perf_counter() - t0) / (tokens * layers)
    per_token = per_layer * W.LLAMA_7B.n_layers
    return {"value": 1.0 / per_token, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "weight_GBps": W.LLAMA_7B.layer_bytes() * W.LLAMA_7B.n_layers / per_token / 1e9,
            "sample": f"the same decoder's batch-1 decode in PyTorch bf16 on the host cores (the reference's "
                      f"forward with no GPU): {layers} 7B-shape layers x {tokens} tokens at context {context}, "
                      "scaled linearly to 32 layers"}


def bench_dit(budget_gb: float, tokens: int, text: int, steps: int, copy_engine: str = "auto") -> dict:
    """One Wan-style DiT denoising step, all 40 blocks resident, then streamed under ``budget_gb``.

    The resident step is measured with the whole model on the GPU (28 GB of
    HBM), then the same weights go back to the host, are offloaded under the
    budget and the streamed step is measured; its output is compared bitwise
    with the resident one.
    """
    import gc

    import torch

    from flextensor_amd import workloads as W
    from flextensor_amd.config import OffloadConfig
    from flextensor_amd.manager import OffloadManager

    dev = torch.device("cuda", 0)
    S = W.WAN_DIT
    model = W.build_dit(S, seed=0, init_device="cuda")
    x, e, ctx = W.dit_inputs(S, tokens, text, seed=0, device="cuda")
    model.to(dev)
    with torch.no_grad():
        want = model(x, e, ctx)  # warm-up and the reference output
        resident_times = []
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model(x, e, ctx)
            torch.cuda.synchronize()
            resident_times.append(time.perf_counter() - t0)
    model.to("cpu")
    gc.collect()
    torch.cuda.empty_cache()
    resident_step = sum(resident_times) / len(resident_times)
    mgr = OffloadManager("bench-dit")
    mgr.offload(model, OffloadConfig(include_patterns=["blocks.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                                     profiling_iters=1, max_gpu_mem_bytes=int(budget_gb * 1e9),
                                     offload_timing="eager", copy_engine=copy_engine))
    with torch.no_grad():
        # discovery and profiling on the full step: the copy engine is chosen from the profiled compute
        model(x, e, ctx)
        model(x, e, ctx)
        got = model(x, e, ctx)  # warm-up step
        mgr.reset_offload_timing()
        step_times = []
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model(x, e, ctx)
            torch.cuda.synchronize()
            step_times.append(time.perf_counter() - t0)
    bitwise = bool(torch.equal(got, want))
    rep = mgr.collect_offload_timing()
    plan = mgr.plan
    streamed = sum(mgr._unit(b).nbytes for b in plan.streamed)
    step = sum(step_times) / len(step_times)
    out = {
        "tokens": tokens, "text_tokens": text, "blocks": S.n_blocks,
        "streamed_blocks": len(plan.streamed), "resident_blocks": len(plan.resident),
        "step_s": step, "resident_step_s": resident_step, "overhead_vs_resident": step / resident_step - 1.0,
        "bitwise_equal_to_resident": bitwise,
        "hidden_fraction": rep.hidden_fraction,
        "transfer_ms_per_step": rep.total_transfer_sum / rep.num_passes,
        "wait_ms_per_step": rep.total_wait_sum / rep.num_passes,
        "link_GBps_during_transfer": streamed / (rep.total_transfer_sum / rep.num_passes * 1e-3) / 1e9,
        "streamed_bytes_per_step": streamed,
        "timed_steps": steps, "streamed_block_bytes": sorted({mgr._unit(b).nbytes for b in plan.streamed}),
        "tflops_per_step": S.block_flops(tokens, text) * S.n_blocks / 1e12,
        "achieved_tflops": S.block_flops(tokens, text) * S.n_blocks / step / 1e12,
        "gpu_weight_bytes": mgr.get_gpu_memory_usage().total_bytes, "budget_bytes": int(budget_gb * 1e9),
        "copy_policy": None if mgr.link is None else {k: mgr.link.to_dict()[k] for k in (
            "kernel_max_bytes", "n_copy_streams", "kernel_grid", "link_bound", "pass_compute_ms",
            "pass_transfer_ms")},
    }
    mgr.release(preserve_model=False)
    del want, got
    return out


def hbm_read_probe(sizes_mib=(512, 2048, 8192), grids=(1024, 2048, 4096), reps: int = 10) -> dict:
    """Plain streaming read rate of HBM (``ftx_hbm_read_probe``): the practical ceiling the HBM-bound
    kernels are compared with. Best of ``reps`` reads per size and grid, HIP events on the stream."""
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HipEvent, current_stream

    dev = torch.device("cuda", 0)
    s = current_stream(dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out: dict = {"GBps": {}}
    for mib in sizes_mib:
        buf = torch.empty(mib * MiB, dtype=torch.uint8, device=dev)
        buf.random_(0, 256)
        row = {}
        for grid in grids:
            best = float("inf")
            for _ in range(reps + 1):
                a, b = HipEvent(True), HipEvent(True)
                s.record_event(a)
                nat.call("ftx_hbm_read_probe", buf.data_ptr(), buf.numel(), sink.data_ptr(), grid, s.handle)
                s.record_event(b)
                b.synchronize()
                best = min(best, a.elapsed_time(b))
            row[str(grid)] = round(buf.numel() / best / 1e6, 1)
        out["GBps"][str(mib)] = row
        del buf
    out["best_GBps"] = max(v for row in out["GBps"].values() for v in row.values())
    out["frac_of_8TBps"] = round(out["best_GBps"] / HBM_PEAK_GBPS, 4)
    return out


def _mem_available_bytes() -> int:
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except OSError:
        pass
    return 0


def bench_llama70b_fp8(budget_gb: float, batch: int, prompt_len: int, decode: int, layers: int,
                       ring_order: str = "auto") -> dict:
    """Batch decode of the 70B-shape decoder with fp8 weights (per-channel bf16 scales) under a GPU budget."""
    import torch

    from flextensor_amd import workloads as W
    from flextensor_amd.config import OffloadConfig
    from flextensor_amd.manager import OffloadManager

    s = W.LlamaShape(**{**W.LLAMA_70B_FP8.__dict__, "n_layers": layers})
    need = s.layer_bytes() * s.n_layers * 2 + (8 << 30)
    avail = _mem_available_bytes()
    if avail < need:
        return {"skipped": f"needs ~{need / 2**30:.0f} GiB of host memory, {avail / 2**30:.0f} GiB available"}
    dev = torch.device("cuda", 0)
    t0 = time.perf_counter()
    model = W.build_llama(s, seed=3, init_device="cuda")
    t_build = time.perf_counter() - t0
    mgr = OffloadManager("bench-70b")
    t0 = time.perf_counter()
    # Module order is the execution order of this decoder, so no discovery pass. One profiled pass, a batch
    # decode token like the timed ones, gives the measured pass rule the compute it weighs against the link.
    mgr.offload(model, OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=0,
                                     profiling_iters=1, max_gpu_mem_bytes=int(budget_gb * 1e9)))
    prompt = W.prompt_tokens(batch, prompt_len, s.vocab, seed=3).to(dev)
    model.init_cache(batch, prompt_len + decode + 2, dev)
    with torch.no_grad():
        model(prompt[:, :1], 0)  # the profiling pass; the plan, the copy policy and the loader are built after it
    torch.cuda.synchronize()
    t_setup = time.perf_counter() - t0
    _log(f"70b: built {t_build:.1f} s, profiled and streaming set up {t_setup:.1f} s; "
         f"{len(mgr.plan.streamed)} streamed / {len(mgr.plan.resident)} resident layers; "
         f"{mgr.link.describe() if mgr.link is not None else 'default copy policy'}")
    _set_ring_order(mgr, ring_order)
    model.init_cache(batch, prompt_len + decode + 2, dev)
    with torch.no_grad():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = model(prompt, 0)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        tok = logits.argmax(-1)
        pos = prompt_len
        model(tok, pos)  # warm-up step
        pos += 1
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(decode):
            tok = model(tok, pos).argmax(-1)
            pos += 1
        torch.cuda.synchronize()
        t_step = (time.perf_counter() - t0) / decode
    streamed = sum(mgr._unit(x).nbytes for x in mgr.plan.streamed)
    out = {
        "layers": s.n_layers, "batch": batch, "prompt_tokens": prompt_len, "decode_steps": decode,
        "streamed_layers": len(mgr.plan.streamed), "resident_layers": len(mgr.plan.resident),
        "layer_bytes": s.layer_bytes(), "streamed_bytes_per_step": streamed,
        "step_s": t_step, "decode_tok_s": batch / t_step, "decode_effective_GBps": streamed / t_step / 1e9,
        "prefill_s": t_prefill, "gpu_weight_bytes": mgr.get_gpu_memory_usage().total_bytes,
        "budget_bytes": int(budget_gb * 1e9), "setup_s": t_setup,
        "copy_policy": None if mgr.link is None else {k: mgr.link.to_dict()[k] for k in (
            "kernel_max_bytes", "n_copy_streams", "kernel_grid", "link_bound", "pass_compute_ms",
            "pass_transfer_ms")},
        "ring_copy_engine": _ring_engine(mgr),
        "ring_order": _ring_order(mgr),
    }
    mgr.release(preserve_model=False)
    return out


def bench_fp8_linear(batch: int = 8, reps: int = 20) -> dict:
    """HBM roofline of the fp8-weight MFMA linear on one 70B-shape decoder layer's projections.

    Every projection has its own weights (858 MB per layer, more than the
    256 MB Infinity Cache, so no call finds the previous call's weights
    cached). The layer runs as the decoder runs it: grouped calls for q/k/v
    and for gate/up, single calls for o and down, each the main kernel plus,
    when K is split, one reduce launch. Algorithmic bytes per call = fp8
    weights (n*k) + bf16 activations (m*k*2) + bf16 outputs (m*n*2) + bf16
    scales (n*2). GPU time: ``reps`` layers captured in one HIP graph (two
    layers' weights alternated), one replay timed with HIP events on the
    replay stream, so host overhead is excluded. Each call is also timed the
    same way on its own. One call per projection (no grouping) and the
    dequantize-then-GEMM forward are timed beside them.
    """
    import torch
    import torch.nn.functional as F

    from flextensor_amd import hip
    from flextensor_amd import workloads as W

    s = W.LLAMA_70B_FP8
    h, q, kv, it = s.hidden, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim, s.inter
    projections = [("wq", q, h), ("wk", kv, h), ("wv", kv, h), ("wo", h, q), ("gate", it, h), ("up", it, h),
                   ("down", h, it)]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(3)
    n_layers = 2  # two layers' weights, alternated, so consecutive layers never share a weight byte
    layers = []
    for _ in range(n_layers):
        layer = {}
        for name, n, k in projections:
            w = (torch.randn(n, k, device=dev, generator=gen) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
            sc = (torch.rand(n, device=dev, generator=gen) / 448).to(torch.bfloat16)
            layer[name] = (w, sc)
        layers.append(layer)
    xs = {k: torch.randn(batch, k, device=dev, generator=gen).to(torch.bfloat16) for k in (h, it)}
    calls = [("qkv", ("wq", "wk", "wv"), h), ("o", ("wo",), q), ("gate+up", ("gate", "up"), h), ("down", ("down",), it)]

    def run_call(layer, names, k):
        if len(names) == 1:
            w, sc = layer[names[0]]
            return [hip.fp8_linear(xs[k], w, sc)]
        return hip.fp8_linear_group(xs[k], [layer[nm][0] for nm in names], [layer[nm][1] for nm in names])

    def graph_ms(fn, n):
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(0)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for i in range(n):
                    fn(i)
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            a.record(side)
            graph.replay()
            b.record(side)
        torch.cuda.synchronize()
        del graph
        return a.elapsed_time(b) / n

    rows = {name: n for name, n, _ in projections}

    def nbytes(names, k):
        return sum(rows[nm] * k + batch * rows[nm] * 2 + rows[nm] * 2 for nm in names) + batch * k * 2

    layer_bytes = sum(nbytes(names, k) for _, names, k in calls)
    layer_ms = graph_ms(lambda i: [run_call(layers[i % n_layers], names, k) for _, names, k in calls], reps)
    # The same projections with the operations that consume their outputs, as the decoder runs them: the
    # residual add after o and after down, SiLU(gate) * up before down (whose input it is). Separately
    # (torch's bf16 ops after each call), then with those ops folded into the calls' reduce kernels.
    resid = torch.randn(batch, h, device=dev, generator=gen).to(torch.bfloat16)

    def path_separate(i):
        lay = layers[i % n_layers]
        run_call(lay, ("wq", "wk", "wv"), h)
        h1 = resid + hip.fp8_linear(xs[q], *lay["wo"])
        g, u = run_call(lay, ("gate", "up"), h)
        return h1 + hip.fp8_linear(F.silu(g) * u, *lay["down"])

    def path_fused(i):
        lay = layers[i % n_layers]
        run_call(lay, ("wq", "wk", "wv"), h)
        h1 = hip.fp8_linear_residual(xs[q], *lay["wo"], resid)
        act = hip.fp8_linear_swiglu(xs[h], *lay["gate"], *lay["up"])
        return hip.fp8_linear_residual(act, *lay["down"], h1)

    separate_ms = graph_ms(path_separate, reps)
    fused_ms = graph_ms(path_fused, reps)
    path_err = float((path_fused(0).double() - path_separate(0).double()).norm() / path_separate(0).double().norm())
    per_call = []
    for label, names, k in calls:
        ms = graph_ms(lambda i, names=names, k=k: run_call(layers[i % n_layers], names, k), reps)
        nb = nbytes(names, k)
        ws = hip.fp8_linear_group_workspace_bytes(batch, [rows[nm] for nm in names], k)
        per_call.append({"call": label, "matrices": list(names), "k": k, "us": round(ms * 1e3, 2),
                         "GBps": round(nb / ms / 1e6, 1), "algorithmic_bytes": nb,
                         "k_slices": ws // (4 * batch * sum(rows[nm] for nm in names)) or 1})
    ungrouped_ms = graph_ms(lambda i: [hip.fp8_linear(xs[k], *layers[i % n_layers][nm]) for nm, _, k in projections], reps)
    # accuracy of every output against float32, and the dequantize-then-GEMM forward it replaces
    errs = {}
    dq_ms = 0.0
    for label, names, k in calls:
        outs = run_call(layers[0], names, k)
        for nm, y in zip(names, outs):
            w, sc = layers[0][nm]
            want = (xs[k].float() @ w.float().t()) * sc.float()
            errs[nm] = round(float((y.float() - want).norm() / want.norm()), 5)
            del want
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            F.linear(xs[k], w.to(torch.bfloat16)) * sc
            a.record()
            for _ in range(3):
                F.linear(xs[k], w.to(torch.bfloat16)) * sc
            b.record()
            torch.cuda.synchronize()
            dq_ms += a.elapsed_time(b) / 3
    big = max(per_call, key=lambda c: c["algorithmic_bytes"])
    achieved = layer_bytes / layer_ms / 1e6
    del layers
    torch.cuda.empty_cache()
    # the same four launches as plain streaming reads of each call's bytes (ftx_hbm_read_probe), two sets of
    # buffers alternated as the layers are: what HBM gives this launch structure with no compute at all
    from flextensor_amd import _native as nat

    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    sizes = [(nbytes(names, k) + 15) // 16 * 16 for _, names, k in calls]
    bufs = [[torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 256) for n in sizes] for _ in range(n_layers)]

    def read_layer(i):
        stream = torch.cuda.current_stream().cuda_stream
        for buf in bufs[i % n_layers]:
            nat.call("ftx_hbm_read_probe", buf.data_ptr(), buf.numel(), sink.data_ptr(), 2048, stream)

    read_ms = graph_ms(read_layer, reps)
    del bufs
    torch.cuda.empty_cache()
    return {"batch": batch, "calls": per_call, "layer_us": round(layer_ms * 1e3, 2),
            "decoder_path": {
                "what": "the four calls with their consumers: residual adds after o and down, SiLU(gate)*up "
                        "feeding down",
                "separate_us": round(separate_ms * 1e3, 2), "fused_us": round(fused_ms * 1e3, 2),
                "frac_separate": round(layer_bytes / separate_ms / 1e6 / HBM_PEAK_GBPS, 4),
                "frac_fused": round(layer_bytes / fused_ms / 1e6 / HBM_PEAK_GBPS, 4),
                "fused_vs_separate_rel_err": round(path_err, 6)},
            "plain_read_layer_us": round(read_ms * 1e3, 2),
            "frac_of_plain_read": round(read_ms / layer_ms, 4),
            "layer_ungrouped_us": round(ungrouped_ms * 1e3, 2), "layer_dequant_gemm_us": round(dq_ms * 1e3, 2),
            "rel_err_vs_fp32": errs, "timing": f"HIP graph of {reps} layers (two layers' weights alternated), one replay",
            "roofline": {"kernel": "fp8_linear_kernel + fp8_linear_reduce_kernel (grouped q/k/v and gate/up)",
                         "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBPS, 4), "algorithmic_bytes_per_layer": int(layer_bytes),
                         "per": "decoder layer (4 calls)"},
            "roofline_largest_call": {"call": big["call"], "achieved": big["GBps"], "peak": HBM_PEAK_GBPS,
                                      "unit": "GB/s", "frac": round(big["GBps"] / HBM_PEAK_GBPS, 4)}}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def bench_fp8_prefill(rows: int = 512, reps: int = 5) -> dict:
    """The fp8 prefill kernel (tiled MFMA GEMM) on one 70B-shape layer's projections at ``rows`` activation rows
    (batch 8 x 64 prompt tokens), as the decoder runs them (grouped q/k/v and gate/up, single o and down).

    Compute-bound: 2 * rows * n * k flops per matrix, against the dense bf16 MFMA peak. GPU time from a HIP
    graph of ``reps`` layers (two layers' weights alternated); the dequantize-then-bf16-GEMM forward it
    replaces is timed beside it."""
    import torch
    import torch.nn.functional as F

    from flextensor_amd import hip
    from flextensor_amd import workloads as W

    s = W.LLAMA_70B_FP8
    h, q, kv, it = s.hidden, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim, s.inter
    rows_of = {"wq": q, "wk": kv, "wv": kv, "wo": h, "gate": it, "up": it, "down": h}
    calls = [("qkv", ("wq", "wk", "wv"), h), ("o", ("wo",), q), ("gate+up", ("gate", "up"), h), ("down", ("down",), it)]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(3)
    layers = []
    for _ in range(2):
        layer = {}
        for _, names, k in calls:
            for nm in names:
                w = (torch.randn(rows_of[nm], k, device=dev, generator=gen) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
                layer[nm] = (w, (torch.rand(rows_of[nm], device=dev, generator=gen) / 448).to(torch.bfloat16))
        layers.append(layer)
    xs = {k: torch.randn(rows, k, device=dev, generator=gen).to(torch.bfloat16) for k in (h, it)}

    def run(layer, names, k):
        if len(names) == 1:
            return [hip.fp8_linear(xs[k], *layer[names[0]])]
        return hip.fp8_linear_group(xs[k], [layer[nm][0] for nm in names], [layer[nm][1] for nm in names])

    def graph_ms(fn, n):
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(0)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for i in range(n):
                    fn(i)
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            a.record(side)
            graph.replay()
            b.record(side)
        torch.cuda.synchronize()
        del graph
        return a.elapsed_time(b) / n

    flops = {label: sum(2.0 * rows * rows_of[nm] * k for nm in names) for label, names, k in calls}
    layer_ms = graph_ms(lambda i: [run(layers[i % 2], names, k) for _, names, k in calls], reps)
    per_call = []
    for label, names, k in calls:
        ms = graph_ms(lambda i, names=names, k=k: run(layers[i % 2], names, k), reps)
        per_call.append({"call": label, "us": round(ms * 1e3, 1), "TFLOPs": round(flops[label] / ms / 1e9, 1)})
    errs, dq_ms = {}, 0.0
    for label, names, k in calls:
        for nm, y in zip(names, run(layers[0], names, k)):
            w, sc = layers[0][nm]
            want = (xs[k].float() @ w.float().t()) * sc.float()
            errs[nm] = round(float((y.float() - want).norm() / want.norm()), 5)
            del want
            F.linear(xs[k], w.to(torch.bfloat16)) * sc
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(3):
                F.linear(xs[k], w.to(torch.bfloat16)) * sc
            b.record()
            torch.cuda.synchronize()
            dq_ms += a.elapsed_time(b) / 3
    # hipBLASLt's bf16 GEMM on weights already dequantized to bf16 (twice the
    # weight bytes, no conversion), timed the same way: the library reference point
    bf16_layers = [{nm: (w.to(torch.bfloat16), sc) for nm, (w, sc) in layer.items()} for layer in layers]

    def run_bf16(layer, names, k):
        return [F.linear(xs[k], layer[nm][0]) * layer[nm][1] for nm in names]

    bf16_ms = graph_ms(lambda i: [run_bf16(bf16_layers[i % 2], names, k) for _, names, k in calls], reps)
    del bf16_layers
    total = sum(flops.values())
    achieved = total / layer_ms / 1e9
    del layers
    torch.cuda.empty_cache()
    ceiling = mfma_probe()
    return {"rows": rows, "calls": per_call, "layer_us": round(layer_ms * 1e3, 1),
            "layer_dequant_gemm_us": round(dq_ms * 1e3, 1),
            "layer_bf16_gemm_predequantized_us": round(bf16_ms * 1e3, 1), "rel_err_vs_fp32": errs,
            "mfma_probe": ceiling,
            "roofline": {"kernel": "fp8_prefill_kernel", "bound": "mfma", "achieved": round(achieved, 1),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "flops_per_layer": total,
                         "frac_of_measured_mfma_rate": round(achieved / ceiling["best_TFLOPs"], 4),
                         "frac_of_measured_16x16x32_rate": round(achieved / ceiling["best_TFLOPs_16x16x32"], 4)}}


def mfma_probe(per_cu=(1, 2, 4), iters: int = 8192, reps: int = 3) -> dict:
    """Sustained MFMA rate (``ftx_mfma_probe_shape``): independent v_mfma_f32_16x16x32_bf16 (the prefill
    kernel's instruction) and v_mfma_f32_32x32x16_bf16 on random bf16 operands that change every MFMA, at 1, 2
    and 4 workgroups of 4 waves per CU; best of ``reps`` per case, HIP events. The better instruction's best is
    the practical ceiling the compute-bound kernels are compared with (the 2.5 PFLOP/s peak is nominal)."""
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HipEvent, current_stream

    dev = torch.device("cuda", 0)
    s = current_stream(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    out: dict = {"TFLOPs": {}, "TFLOPs_32x32x16": {}}
    for shape, key in ((0, "TFLOPs"), (1, "TFLOPs_32x32x16")):
        for n in per_cu:
            wgs = n * cus
            flops = 2.0 * 16 * 16 * 32 * 32 * iters * 4 * wgs  # both shapes: 524288 flops per wave iteration
            best = float("inf")
            for _ in range(reps + 1):
                a, b = HipEvent(True), HipEvent(True)
                s.record_event(a)
                nat.call("ftx_mfma_probe_shape", shape, wgs, iters, sink.data_ptr(), s.handle)
                s.record_event(b)
                b.synchronize()
                best = min(best, a.elapsed_time(b))
            out[key][f"{n}_workgroups_per_cu"] = round(flops / best / 1e9, 1)
    out["best_TFLOPs_16x16x32"] = max(out["TFLOPs"].values())
    out["best_TFLOPs"] = max(out["best_TFLOPs_16x16x32"], max(out["TFLOPs_32x32x16"].values()))
    out["frac_of_nominal_peak"] = round(out["best_TFLOPs"] / MFMA_BF16_PEAK_TFLOPS, 4)
    return out


def staged_sweep(repeats: int = 5) -> dict:
    """Host-to-device GB/s from pageable memory: the staged engine by threads and piece size.

    Sources: an ordinary pageable allocation and a POSIX shared-memory mapping
    (the blocks a shared-offload follower streams from). Beside them:
    ``hipMemcpyAsync`` straight from the pageable source (the runtime's own
    staging) and from pinned memory (the link's peak). Each figure is the best
    of ``repeats`` copies of 512 MiB, timed on the host around the call plus a
    stream synchronize (the staged copy works on the host while the link runs).
    """
    import uuid

    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HostArena, current_stream
    from flextensor_amd.shm import SharedSegment

    dev = torch.device("cuda", 0)
    n = 512 * MiB
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    s = current_stream(dev)
    pageable = torch.randint(0, 256, (n,), dtype=torch.uint8)
    seg = SharedSegment(f"ftbench_{uuid.uuid4().hex[:8]}", n, create=True)
    shm = torch.frombuffer(seg.buf, dtype=torch.uint8)
    shm.copy_(pageable)
    pinned = HostArena(n)
    pinned.tensor.copy_(pageable)

    def best(src: torch.Tensor, mode: int) -> float:
        times = []
        for _ in range(repeats + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            nat.copy_h2d(dst.data_ptr(), src.data_ptr(), n, mode, s.handle)
            s.synchronize()
            times.append(time.perf_counter() - t0)
        return n / min(times[1:]) / 1e9

    piece0, threads0 = nat.get_staging_policy()
    out: dict = {"bytes": n, "pinned_sdma_GBps": round(best(pinned.tensor, nat.COPY_SDMA), 2),
                 "pageable_hipMemcpyAsync_GBps": round(best(pageable, nat.COPY_SDMA), 2), "staged": []}
    try:
        for piece_mib in (8, 32, 64):
            for threads in (1, 2, 4, 8, 16):
                nat.set_staging_policy(piece_mib * MiB, threads)
                out["staged"].append({"piece_MiB": piece_mib, "threads": threads,
                                      "pageable_GBps": round(best(pageable, nat.COPY_STAGED), 2),
                                      "shm_GBps": round(best(shm, nat.COPY_STAGED), 2)})
                _log(f"staged {piece_mib} MiB x {threads} threads: {out['staged'][-1]}")
    finally:
        nat.set_staging_policy(piece0, 0)
        ok = torch.equal(dst.cpu(), pageable)
        del shm
        seg.unlink()
    out["last_copy_bit_exact"] = bool(ok)
    out["default_policy"] = {"piece_MiB": piece0 // MiB, "threads": threads0}
    return out


def cpu_llama70b_decode_baseline(batch: int = 8, context: int = 64, steps: int = 2) -> dict:
    """Batch decode of one 70B-shape layer in PyTorch on the host cores, scaled to 80 layers.

    torch has no fp8 GEMM on the CPU, so the layer holds bf16 weights, which
    is what dequantizing the fp8 weights on the host gives.
    """
    import torch

    from flextensor_amd import workloads as W

    s = W.LlamaShape(**{**W.LLAMA_70B_FP8.__dict__, "n_layers": 1, "vocab": 256, "fp8": False,
                        "max_seq": context + steps + 4})
    model = W.build_llama(s, seed=3)
    model.init_cache(batch, context + steps + 4, torch.device("cpu"))
    layer = model.layers[0]
    x = torch.randn(batch, 1, s.hidden, dtype=torch.bfloat16)
    with torch.no_grad():
        layer(x, context, model.rope_cos, model.rope_sin, model.cache_k[0], model.cache_v[0])  # warm-up
        t0 = time.perf_counter()
        for i in range(steps):
            layer(x, context + 1 + i, model.rope_cos, model.rope_sin, model.cache_k[0], model.cache_v[0])
        per_layer = (time.perf_counter() - t0) / steps
    per_step = per_layer * W.LLAMA_70B_FP8.n_layers
    return {"value": batch / per_step, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"PyTorch bf16 (fp8 dequantized) batch-{batch} decode of one 70B-shape layer x {steps} steps "
                      f"at context {context}, scaled linearly to 80 layers"}


RING_COPY_PROBES = 3  # ring copies of one 7B-shape decoder layer in the traffic probe


def measure_traffic(args) -> dict | None:
    """HBM bytes per scatter launch, per ring copy and per encoded-block decode from two ``rocprofv3 --pmc``
    child runs.

    Each child runs this script in ``--traffic-probe`` mode: one 1 GiB
    device-to-device copy (the runtime's copy kernel, whose traffic is known:
    1 GiB read, 1 GiB written), then one step of the scatter workload, then
    ``RING_COPY_PROBES`` ring copies of one 7B-shape decoder layer (404,766,720
    B from a page-locked arena) on the zero-copy kernel at the link-bound
    grid, as the headline decode copies them. The counter reading of the
    calibration copy gives the scale of each counter; traffic = scaled
    FETCH_SIZE + scaled WRITE_SIZE, averaged over the scatter launches. For the
    ring copy FETCH_SIZE counts the bytes read from host memory over the link
    and WRITE_SIZE the bytes written to HBM (``ring_copy``). The child then
    decodes the same layer's bytes, as N(0, 0.02) bf16 weights exponent-coded,
    ``RING_COPY_PROBES`` times (``expcode_decode``: the encoded bytes read over
    the link, the raw bytes written). Returns None when rocprofv3 is not
    available or a pass fails.
    """
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile

    from flextensor_amd import link_model as L

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    calib = 1024 * MiB
    out: dict = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix=f"ftx_pmc_{ctr.lower()}_", dir="/tmp")
        cmd = [exe, "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "pmc", "--", sys.executable,
               os.path.abspath(__file__), "--traffic-probe", "--chunk-mib", str(args.chunk_mib),
               "--tensors", str(args.tensors), "--copy-engine", args.copy_engine]
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), capture_output=True, text=True,
                               timeout=300)
        except subprocess.TimeoutExpired:
            _log(f"traffic: rocprofv3 {ctr} pass timed out")
            return None
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if r.returncode != 0 or not files:
            _log(f"traffic: rocprofv3 {ctr} pass failed (rc {r.returncode}): {r.stderr[-400:]}")
            return None
        with open(files[0]) as fh:
            rows = sorted(csv.DictReader(fh), key=lambda row: int(row["Dispatch_Id"]))
        copies = [row for row in rows if row["Kernel_Name"] == "__amd_rocclr_copyBuffer"]
        scat = [row for row in rows if "scatter_kernel" in row["Kernel_Name"]]
        ring = [row for row in rows if "zero_copy_kernel" in row["Kernel_Name"]
                and int(row.get("Grid_Size", L.RING_KERNEL_GRID * 256)) == L.RING_KERNEL_GRID * 256]
        dec = [row for row in rows if "expcode_dense_link_decode_kernel" in row["Kernel_Name"]]
        if not copies or not scat:
            return None
        scale = calib / (float(copies[0]["Counter_Value"]) * 1024)

        def per_launch(sel: list, want: int | None = None) -> float | None:
            if not sel or (want is not None and len(sel) != want):
                return None
            return sum(float(row["Counter_Value"]) for row in sel) * 1024 * scale / len(sel)

        out[ctr] = {"scale": round(scale, 4), "bytes_per_launch": per_launch(scat),
                    "ring_bytes_per_launch": per_launch(ring, RING_COPY_PROBES),
                    "decode_bytes_per_launch": per_launch(dec, RING_COPY_PROBES)}
        for line in r.stdout.splitlines():
            if line.startswith("expcode_encoded_bytes "):
                out["expcode_encoded_bytes"] = int(line.split()[1])
        shutil.rmtree(d, ignore_errors=True)
    res = {"traffic": out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"],
           "fetch_bytes_per_launch": out["FETCH_SIZE"]["bytes_per_launch"],
           "write_bytes_per_launch": out["WRITE_SIZE"]["bytes_per_launch"],
           "fetch_scale": out["FETCH_SIZE"]["scale"], "write_scale": out["WRITE_SIZE"]["scale"]}
    if out["FETCH_SIZE"]["ring_bytes_per_launch"] is not None and out["WRITE_SIZE"]["ring_bytes_per_launch"] is not None:
        res["ring_copy"] = {"host_read_bytes_per_launch": out["FETCH_SIZE"]["ring_bytes_per_launch"],
                            "hbm_write_bytes_per_launch": out["WRITE_SIZE"]["ring_bytes_per_launch"]}
    if (out["FETCH_SIZE"]["decode_bytes_per_launch"] is not None
            and out["WRITE_SIZE"]["decode_bytes_per_launch"] is not None):
        res["expcode_decode"] = {"host_read_bytes_per_launch": out["FETCH_SIZE"]["decode_bytes_per_launch"],
                                 "hbm_write_bytes_per_launch": out["WRITE_SIZE"]["decode_bytes_per_launch"],
                                 "encoded_bytes_per_launch": out.get("expcode_encoded_bytes")}
    return res


def traffic_probe(args) -> int:
    import torch

    src = torch.ones(1024 * MiB, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    bench_scatter(1, 0, args.chunk_mib, args.tensors, args.copy_engine, verify=False)
    from flextensor_amd import _native as nat
    from flextensor_amd import link_model as L
    from flextensor_amd import workloads as W
    from flextensor_amd.hip import HostArena, transfer_stream

    n = W.LLAMA_7B.layer_bytes()
    arena = HostArena(n)
    slot = torch.empty(n, dtype=torch.uint8, device="cuda")
    xs = transfer_stream(torch.device("cuda", 0))
    ring_policy = nat.copy_policy(n, 2**63 - 1, 1, L.RING_KERNEL_GRID)
    for _ in range(RING_COPY_PROBES):
        nat.copy_h2d(slot.data_ptr(), arena.ptr, n, nat.COPY_KERNEL, xs.handle, ring_policy)
    xs.synchronize()
    # the same layer's bytes as N(0, 0.02) bf16 weights, in the dense format, decoded as the encoded ring does
    from flextensor_amd import expcode

    g = torch.Generator().manual_seed(0)
    arena.tensor[:n].copy_((torch.randn(n // 2, generator=g) * 0.02).to(torch.bfloat16).view(torch.uint8))
    block = expcode.encode(arena.tensor[:n], dense=True)
    for _ in range(RING_COPY_PROBES):
        expcode.decode_h2d(slot, block, stream=xs)
    xs.synchronize()
    print(f"expcode_encoded_bytes {block.nbytes}", flush=True)
    return 0


def copy_behind_fp8(reps: int = 5) -> dict:
    """How long a reserved-CU ring copy waits when it is queued behind a running LDS-heavy fp8 grid.

    A copy grid of at most 16 workgroups asks for each CU's whole LDS, so it
    cannot start on a CU where a workgroup that uses LDS is resident. Here the
    grouped gate/up projections of a 70B-shape layer run on the compute
    stream, once at 512 rows (the prefill kernel) and once at 8 rows (the
    decode kernel and its reduce). A 64 MiB zero-copy copy at 8 workgroups is
    queued on the transfer stream as the GEMM starts. Device timestamps
    (``ftx_timestamp``) bracket both; medians of ``reps``. The copy's start
    delay is its bracketed time beside the GEMM minus its time alone.
    """
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd import hip
    from flextensor_amd import link_model as L
    from flextensor_amd import workloads as W

    dev = torch.device("cuda", 0)
    comp, xs = hip.current_stream(dev), hip.transfer_stream(dev)
    s = W.LLAMA_70B_FP8
    gen = torch.Generator(device=dev).manual_seed(5)
    ws = [(torch.randn(s.inter, s.hidden, device=dev, generator=gen) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
          for _ in range(2)]
    scs = [(torch.rand(s.inter, device=dev, generator=gen) / 448).to(torch.bfloat16) for _ in range(2)]
    n = 64 * MiB
    arena = hip.HostArena(n)
    arena.tensor.random_(0, 256)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    policy = nat.copy_policy(0, 2**63 - 1, 1, L.RING_KERNEL_GRID)

    def copy(stream):
        nat.copy_h2d(dst.data_ptr(), arena.ptr, n, nat.COPY_KERNEL, stream.handle, policy)

    out: dict = {"copy_bytes": n, "copy_workgroups": L.RING_KERNEL_GRID}
    for label, rows in (("prefill_gate_up_512_rows", 512), ("decode_gate_up_8_rows", 8)):
        x = torch.randn(rows, s.hidden, device=dev, generator=gen).to(torch.bfloat16)
        hip.fp8_linear_group(x, ws, scs)  # warm-up, and the workspace shape is cached
        copy(xs)
        torch.cuda.synchronize()
        rec: dict[str, list[float]] = {"gemm_alone_us": [], "copy_alone_us": [], "gemm_beside_copy_us": [],
                                       "copy_behind_gemm_us": []}
        for _ in range(reps):
            clock = hip.DeviceClock(8, dev)
            e = [clock.event() for _ in range(8)]
            e[0].record(comp)
            hip.fp8_linear_group(x, ws, scs)
            e[1].record(comp)
            torch.cuda.synchronize()
            e[2].record(xs)
            copy(xs)
            e[3].record(xs)
            torch.cuda.synchronize()
            e[4].record(comp)
            started = comp.record_event()  # reached once the GEMM is dispatched
            hip.fp8_linear_group(x, ws, scs)
            e[5].record(comp)
            xs.wait_event(started)
            e[6].record(xs)
            copy(xs)
            e[7].record(xs)
            torch.cuda.synchronize()
            clock.refresh()
            for key, (a, b) in (("gemm_alone_us", (0, 1)), ("copy_alone_us", (2, 3)),
                                ("gemm_beside_copy_us", (4, 5)), ("copy_behind_gemm_us", (6, 7))):
                rec[key].append(1e3 * e[a].elapsed_time(e[b]))
        row = {k: round(sorted(v)[len(v) // 2], 1) for k, v in rec.items()}
        row["copy_start_delay_us"] = round(row["copy_behind_gemm_us"] - row["copy_alone_us"], 1)
        out[label] = row
        _log(f"copy behind fp8 {label}: {row}")
    return out


def engine_contention() -> dict:
    """How each copy engine shares the GPU with an HBM-bound kernel.

    Three tables, medians of repeated runs on one GPU:

    * host-to-device GB/s of the zero-copy kernel by workgroup count (512 MiB);
    * scatter-kernel time alone, by wave-tile size, for the 512 MiB chunk of
      the 2000-tensor set that holds the most tensors;
    * the same chunk as one descriptor into one buffer, and torch's device
      copy of the same bytes (the plain-copy rate of this HBM);
    * the same scatter (default tile) launched on the compute stream while a
      512 MiB host-to-device copy runs on the transfer stream, per engine.
    """
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd import workloads as W
    from flextensor_amd.hip import HipEvent, HostArena, current_stream, transfer_stream
    from flextensor_amd.scatter import ScatterPlan, _dst_base, plan_chunks

    dev = torch.device("cuda", 0)
    comp, xs = current_stream(dev), transfer_stream(dev)
    n = 512 * MiB
    arena = HostArena(n)
    arena.tensor.random_(0, 256)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)

    def grid_policy(grid):  # each copy carries its grid; the library default stays as it is
        return nat.copy_policy(0, 2**63 - 1, 1, grid)

    def median_ms(fn, stream, reps):
        ts = []
        for _ in range(reps):
            a, b = HipEvent(True), HipEvent(True)
            stream.record_event(a)
            fn()
            stream.record_event(b)
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts)[len(ts) // 2]

    out: dict = {"kernel_grid_GBps": {}, "scatter_alone_us": {}, "scatter_beside_copy_us": {}}
    for grid in (4, 8, 16, 32, 64, 128, 1024):
        pol = grid_policy(grid)
        ms = median_ms(lambda: nat.copy_h2d(dst.data_ptr(), arena.ptr, n, nat.COPY_KERNEL, comp.handle, pol),
                       comp, 5)
        out["kernel_grid_GBps"][grid] = round(n / ms / 1e6, 2)
    sizes = W.scatter_sizes()
    chunk = max(plan_chunks(sizes, 512 * MiB)[:6], key=lambda c: len(c.pieces))
    dests = {p.index: torch.empty(sizes[p.index], dtype=torch.uint8, device=dev) for p in chunk.pieces}
    descs = [(p.chunk_off, _dst_base(dests[p.index]) + p.tensor_off, p.nbytes) for p in chunk.pieces if p.nbytes]
    if any(off + k > chunk.nbytes for off, _, k in descs) or chunk.nbytes > n:
        raise RuntimeError("scatter probe descriptors exceed the chunk")
    payload = sum(k for _, _, k in descs)
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev)
    for tile in (8 << 10, 16 << 10, 32 << 10, 64 << 10):
        plan = ScatterPlan(descs, tile)
        out["scatter_alone_us"][tile] = round(1e3 * median_ms(lambda: plan.run(src, comp), comp, 10), 1)
        plan.close()
    # the same bytes as one descriptor into one buffer, and torch's own device copy: the plain-copy rate
    whole = torch.empty(n, dtype=torch.uint8, device=dev)
    plan = ScatterPlan([(0, whole.data_ptr(), chunk.nbytes)])
    out["scatter_one_descriptor_us"] = round(1e3 * median_ms(lambda: plan.run(src, comp), comp, 10), 1)
    plan.close()
    out["torch_copy_us"] = round(1e3 * median_ms(lambda: whole[:chunk.nbytes].copy_(src[:chunk.nbytes]), comp, 10), 1)
    del whole
    plan = ScatterPlan(descs)
    for label, mode, grid in (("hipMemcpyAsync", nat.COPY_SDMA, 0), ("kernel_grid_1024", nat.COPY_KERNEL, 1024),
                              ("kernel_grid_64", nat.COPY_KERNEL, 64), ("kernel_grid_16", nat.COPY_KERNEL, 16),
                              ("kernel_grid_4", nat.COPY_KERNEL, 4)):
        pol = grid_policy(grid)
        ts = []
        for _ in range(8):
            torch.cuda.synchronize()
            nat.copy_h2d(dst.data_ptr(), arena.ptr, n, mode, xs.handle, pol)
            a, b = HipEvent(True), HipEvent(True)
            comp.record_event(a)
            plan.run(src, comp)
            comp.record_event(b)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        out["scatter_beside_copy_us"][label] = round(1e3 * sorted(ts)[len(ts) // 2], 1)
    plan.close()
    out["scatter_payload_bytes"] = payload
    out["scatter_pieces"] = len(descs)
    del dst, src, arena
    torch.cuda.empty_cache()
    out["copy_queued_behind_fp8"] = copy_behind_fp8()
    return out


def copy_chain(sizes_mib=(90, 386), copies: int = 56, reps: int = 3) -> dict:
    """Idle link time between consecutive ring copies, by what each copy depends on.

    ``copies`` host-to-device copies of B bytes from one pinned arena (two
    halves) into two device slots (a 2-slot ring), on the device's transfer
    stream, the whole chain enqueued at once, in these arrangements:

    * ``back_to_back``: the copies alone, one after another on the transfer stream;
    * ``slot_waits``: before each copy the transfer stream waits on an event the
      compute stream recorded as that slot's release. The compute stream has
      nothing queued, so every wait is already met when the copy is enqueued;
    * ``marks``: an event recorded on the transfer stream after each copy (the
      copy's ready event), which nothing waits on;
    * ``ring``: the streamed pass (loaders.py:1534-1573): the compute stream
      waits for each copy's ready event, reads its slot with a small kernel and
      records the slot's release, which the copy two later waits on;
    * ``consume_only``: the compute stream waits for each ready event and reads
      the slot, but no copy waits on a release (what the compute side costs);
    * ``handshake_only``: the ring's events and waits with no compute kernels
      (what the cross-stream waits cost);
    * ``ring_kernel``: ``ring`` with zero-copy kernel copies at 8 workgroups, the
      link-bound policy;
    * ``*_device_only``: the same with every ready and release event created
      ``device_only`` (``FTX_EVENT_DEVICE_ONLY``: no system-scope fence when
      recorded);
    * ``ring_host_wait`` / ``ring_kernel_host_wait``: the ring with the compute
      stream never waiting on a ready event. The host enqueues two copies ahead,
      then per copy blocks on its ready event, enqueues the slot's read and
      release on the compute stream and the copy two later (behind its release
      wait) on the transfer stream. A copy then has no waiter on another queue
      while it runs.

    Per arrangement and size, the median of ``reps`` chains: microseconds per
    copy (HIP events on the transfer stream around the chain), GB/s, and the
    idle link time per boundary, (chain time - copies x the best single copy)
    / (copies - 1). The best single copy is the fastest of 5 lone copies with
    the same engine.
    """
    import torch

    from flextensor_amd import _native as nat
    from flextensor_amd import link_model as L
    from flextensor_amd.hip import HipEvent, HostArena, current_stream, transfer_stream

    dev = torch.device("cuda", 0)
    comp, xs = current_stream(dev), transfer_stream(dev)
    kernel_policy = nat.copy_policy(0, 2**63 - 1, 1, L.RING_KERNEL_GRID)
    acc = torch.zeros(1, dtype=torch.float32, device=dev)
    kinds = ("back_to_back", "slot_waits", "marks", "marks_device_only", "consume_only", "handshake_only", "ring",
             "ring_device_only", "ring_kernel", "ring_kernel_device_only", "ring_host_wait", "ring_kernel_host_wait")
    out: dict = {"copies": copies, "sizes": {}}
    for mib in sizes_mib:
        nb = mib * MiB
        arena = HostArena(2 * nb)
        arena.tensor.random_(0, 256)
        slots = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(2)]

        def one(slot, mode, policy, stream):
            nat.copy_h2d(slots[slot].data_ptr(), arena.ptr + slot * nb, nb, mode, stream.handle, policy)

        def lone_ms(mode, policy):
            best = float("inf")
            for _ in range(5):
                torch.cuda.synchronize()
                a, b = HipEvent(True), HipEvent(True)
                xs.record_event(a)
                one(0, mode, policy, xs)
                xs.record_event(b)
                b.synchronize()
                best = min(best, a.elapsed_time(b))
            return best

        def host_waited_ms(mode, policy):
            torch.cuda.synchronize()
            ready, released = [None] * copies, [None, None]
            start, end = HipEvent(True), HipEvent(True)
            xs.wait_stream(comp)
            xs.record_event(start)

            def enqueue(i):
                s = i % 2
                if released[s] is not None:
                    xs.wait_event(released[s])
                one(s, mode, policy, xs)
                ready[i] = xs.record_event(HipEvent())

            for i in range(min(2, copies)):
                enqueue(i)
            for i in range(copies):
                ready[i].synchronize()
                acc.add_(slots[i % 2][:4096].float().sum())
                released[i % 2] = comp.record_event(HipEvent())
                if i + 2 < copies:
                    enqueue(i + 2)
            xs.record_event(end)
            torch.cuda.synchronize()
            return start.elapsed_time(end)

        def chain_ms(kind):
            kernel = kind.startswith("ring_kernel")
            mode, policy = (nat.COPY_KERNEL, kernel_policy) if kernel else (nat.COPY_SDMA, None)
            if kind.endswith("_host_wait"):
                return host_waited_ms(mode, policy)
            device_only = kind.endswith("_device_only")
            ring = kind.startswith("ring") or kind == "handshake_only"
            consume = kind.startswith("ring") or kind == "consume_only"
            torch.cuda.synchronize()
            released = [None, None]
            start, end = HipEvent(True), HipEvent(True)
            xs.wait_stream(comp)
            xs.record_event(start)
            for i in range(copies):
                s = i % 2
                if kind == "slot_waits":
                    xs.wait_event(comp.record_event())
                elif ring and released[s] is not None:
                    xs.wait_event(released[s])
                one(s, mode, policy, xs)
                if kind.startswith("marks") or ring or consume:
                    ready = xs.record_event(HipEvent(device_only=device_only))
                    if ring or consume:
                        comp.wait_event(ready)
                        if consume:
                            acc.add_(slots[s][:4096].float().sum())
                        released[s] = comp.record_event(HipEvent(device_only=device_only))
            xs.record_event(end)
            torch.cuda.synchronize()
            return start.elapsed_time(end)

        row: dict = {"bytes": nb}
        lone = {"sdma": lone_ms(nat.COPY_SDMA, None), "kernel_g8": lone_ms(nat.COPY_KERNEL, kernel_policy)}
        row["lone_copy_us"] = {k: round(v * 1e3, 1) for k, v in lone.items()}
        for kind in kinds:
            chain_ms(kind)  # warm-up
            t = sorted(chain_ms(kind) for _ in range(reps))[reps // 2]
            base = lone["kernel_g8" if kind.startswith("ring_kernel") else "sdma"]
            row[kind] = {"us_per_copy": round(t * 1e3 / copies, 1), "GBps": round(copies * nb / t / 1e6, 2),
                         "idle_us_per_boundary": round((t - copies * base) * 1e3 / (copies - 1), 1)}
            _log(f"copy chain {mib} MiB {kind}: {row[kind]}")
        bad = [i for i in range(2) if not torch.equal(slots[i].cpu(), arena.tensor[i * nb:(i + 1) * nb])]
        row["slots_bit_exact"] = not bad
        out["sizes"][str(mib)] = row
        del slots, arena
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed decode tokens of the headline 7B workload")
    ap.add_argument("--warmup", type=int, default=5, help="untimed decode tokens before them")
    ap.add_argument("--chunk-mib", type=int, default=512)
    ap.add_argument("--tensors", type=int, default=2000)
    ap.add_argument("--scatter-steps", type=int, default=5)
    ap.add_argument("--copy-engine", default="auto", choices=["auto", "sdma", "kernel"])
    ap.add_argument("--ring-order", default="auto", choices=["auto", "reference", "link-bound"],
                    help="how the streamed legs order their ring waits (auto: link-bound order in link-bound "
                         "passes)")
    ap.add_argument("--kernel-grid", type=int, default=0,
                    help="zero-copy kernel workgroups for --copy-engine kernel (0: the library default)")
    ap.add_argument("--skip-cpu-baseline", action="store_true")
    ap.add_argument("--budget-gb", type=float, default=8.0)
    ap.add_argument("--prefill", type=int, default=512)
    ap.add_argument("--skip-verify", action="store_true", help="skip the independent byte check of the scatter")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="run one device-to-device copy of this size first (HBM counter calibration)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc traffic passes")
    ap.add_argument("--link-sweep", action="store_true",
                    help="only print the host-to-device GB/s of each copy engine over chunk sizes 64 KiB-512 MiB")
    ap.add_argument("--engine-contention", action="store_true",
                    help="only print how each copy engine shares the GPU with the scatter kernel")
    ap.add_argument("--copy-chain", action="store_true",
                    help="only print the idle link time between chained ring copies, by what each copy waits on")
    ap.add_argument("--hbm-read-probe", action="store_true",
                    help="only print the plain HBM read rate (the ceiling the HBM-bound kernels are compared with)")
    ap.add_argument("--skip-scatter", action="store_true")
    ap.add_argument("--skip-dit", action="store_true")
    ap.add_argument("--skip-mlp", action="store_true")
    ap.add_argument("--skip-finer-units", action="store_true",
                    help="skip the 7B decode with attention and MLP projections as separate offload units")
    ap.add_argument("--encoded-only", action="store_true",
                    help="print only the 7B decode with exponent-coded blocks (for profiling it alone)")
    ap.add_argument("--expcode-sweep", action="store_true",
                    help="print the encoded-block decode of one 7B layer at several grids against raw copies")
    ap.add_argument("--encoded-finer-units", action="store_true",
                    help="with --encoded-only: each layer's attention and MLP projections as separate units")
    ap.add_argument("--no-link-benchmark", action="store_true",
                    help="with --encoded-only: skip the host-link measurement, so the pass regime is not measured "
                         "(for kernel traces, which inflate the profiled compute); pair with --ring-order link-bound")
    ap.add_argument("--encoded-resident", action="store_true",
                    help="with --encoded-only: also keep resident layers exponent-coded in HBM")
    ap.add_argument("--skip-encoded", action="store_true",
                    help="skip the 7B decode with exponent-coded blocks (OffloadConfig.encode_streamed_blocks)")
    ap.add_argument("--skip-70b", action="store_true", help="skip the 80-layer fp8 70B-shape batch-8 decode")
    ap.add_argument("--staged-sweep", action="store_true",
                    help="only print host-to-device GB/s of the staged engine from pageable and shared memory")
    ap.add_argument("--dit-only", action="store_true", help="print only the DiT leg (for profiling it alone)")
    ap.add_argument("--mlp-only", action="store_true",
                    help="print only the 8-layer MLP stack leg (for profiling it alone)")
    ap.add_argument("--fp8-linear-only", action="store_true",
                    help="only print the fp8 linear roofline on the 70B-shape decode projections")
    ap.add_argument("--layers-70b", type=int, default=80)
    ap.add_argument("--dit-tokens", type=int, default=32760)
    ap.add_argument("--dit-steps", type=int, default=2)
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build streams weights into a single MI355X "
              "(multi-GPU sharding is described, not built). Run with --gpus 1.", file=sys.stderr)
        return 2

    import gc

    import torch

    from flextensor_amd import _native as nat

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    nat.load()
    if args.traffic_probe:
        return traffic_probe(args)
    if args.kernel_grid:
        if args.copy_engine != "kernel":
            print("bench: --kernel-grid needs --copy-engine kernel (auto chooses its own grid)", file=sys.stderr)
            return 2
        kmax, smin, nstreams, _ = nat.get_copy_policy()
        nat.set_copy_policy(kmax, smin, nstreams, args.kernel_grid)
    if args.engine_contention:
        print(json.dumps(engine_contention()), flush=True)
        return 0
    if args.copy_chain:
        print(json.dumps({"copy_chain": copy_chain()}), flush=True)
        return 0
    if args.fp8_linear_only:
        print(json.dumps({"fp8_linear": bench_fp8_linear(), "fp8_prefill": bench_fp8_prefill()}), flush=True)
        return 0
    if args.dit_only:
        print(json.dumps({"dit": bench_dit(12.0, args.dit_tokens, 512, args.dit_steps, args.copy_engine)}), flush=True)
        return 0
    if args.expcode_sweep:
        print(json.dumps({"expcode_sweep": expcode_sweep()}), flush=True)
        return 0
    if args.encoded_only:
        peak = measure_link_peak()
        units = FINER_UNITS if args.encoded_finer_units else ("layers.*",)
        enc = bench_llama7b(args.budget_gb, args.prefill, args.steps, args.warmup, args.copy_engine,
                            include_patterns=units, ring_order=args.ring_order, encode=True,
                            encode_resident=args.encoded_resident, link_benchmark=not args.no_link_benchmark)
        enc.pop("_check")
        res = _encoded_summary(enc, max(peak["sdma"], peak["kernel"]), None)
        res["include_patterns"] = list(units)
        key = "llama7b_encoded_resident" if args.encoded_resident else "llama7b_encoded_blocks"
        print(json.dumps({key: res, "measured_peak": peak}), flush=True)
        return 0
    if args.mlp_only:
        res = {"mlp8": bench_mlp(20, args.copy_engine, ring_order=args.ring_order)}
        if not args.skip_encoded:
            res["mlp8_encoded_blocks"] = bench_mlp(20, args.copy_engine, ring_order=args.ring_order, encode=True)
        print(json.dumps(res), flush=True)
        return 0
    if args.staged_sweep:
        print(json.dumps({"staged_sweep": staged_sweep()}), flush=True)
        return 0
    if args.hbm_read_probe:
        print(json.dumps({"hbm_read_probe": hbm_read_probe()}), flush=True)
        return 0
    if args.link_sweep:
        from flextensor_amd.link_model import choose_copy_policy, measure_copy_curve

        sizes = [64 << 10, 256 << 10, 1 << 20, 2 << 20, 4 << 20, 16 << 20, 64 << 20, 180 << 20, 512 << 20]
        curves = {e: measure_copy_curve(e, sizes, repeats=10) for e in ("sdma", "kernel", "sdma_split2")}
        table = {e: {str(n): round(g, 2) for n, g in c.gbps().items()} for e, c in curves.items()}
        policy = choose_copy_policy(curves["sdma"], curves["kernel"], curves["sdma_split2"], 2)
        print(json.dumps({"link_sweep_GBps": table, "auto_policy": {"kernel_max_bytes": policy[0],
                                                                     "split_min_bytes": policy[1],
                                                                     "n_copy_streams": policy[2]}}), flush=True)
        return 0
    if args.calibration_copy_mib:
        src = torch.ones(args.calibration_copy_mib * MiB, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        _log(f"calibration copy: {args.calibration_copy_mib} MiB device to device")
        del src, dst
    peak = measure_link_peak()
    measured_peak = max(peak["sdma"], peak["kernel"])
    _log(f"measured H2D peak (512 MiB, best of 20): sdma {peak['sdma']:.2f} GB/s, kernel {peak['kernel']:.2f} GB/s")

    # ---- headline: 7B-shape decoder, 8 GB budget, one decode token per step
    llama = bench_llama7b(args.budget_gb, args.prefill, args.steps, args.warmup, args.copy_engine,
                          ring_order=args.ring_order)
    check = llama.pop("_check")
    _log(f"llama7b: {llama}")
    line = {
        "metric": "effective streamed-weight GB/s (% of link peak); tok/s at 7B shape, 8 GB budget",
        "value": round(llama["decode_effective_GBps"], 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(llama["ms_per_token"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded random bf16 weights N(0, 0.02), random prompt tokens)",
        "config": {"workload": "Llama-style 32-layer decoder at 7B shape (hidden 4096, 32 heads x 128, SwiGLU 11008, "
                               "RMSNorm, vocab 32000), bf16 weights N(0, 0.02) seed 0; 512-token prefill, then batch-1 "
                               "greedy decode, one step = one decode token; GPU weight budget 8 GB",
                   "model_dtype": "bf16", "budget_bytes": llama["budget_bytes"],
                   "streamed_layers": llama["streamed_layers"], "resident_layers": llama["resident_layers"],
                   "streamed_bytes_per_token": llama["streamed_bytes_per_token"], "copy_engine": args.copy_engine,
                   "copy_policy": llama["copy_policy"], "copy_policy_source": llama["copy_policy_source"],
                   "ring_order": llama["ring_order"], "transfer_stream": llama["transfer_stream"],
                   "encode_streamed_blocks": False},
        "tok_s": round(llama["decode_tok_s"], 3),
        "prefill_tok_s": round(llama["prefill_tok_s"], 1),
        "link": {"decode_effective_GBps": round(llama["decode_effective_GBps"], 3),
                 "measured_peak_GBps": round(measured_peak, 3),
                 "pct_of_measured_peak": round(100 * llama["decode_effective_GBps"] / measured_peak, 2),
                 "pcie_gen5_x16_theoretical_GBps": PCIE_GEN5_X16_GBPS,
                 "pct_of_theoretical": round(100 * llama["decode_effective_GBps"] / PCIE_GEN5_X16_GBPS, 2),
                 "peak_sdma_GBps": round(peak["sdma"], 3), "peak_kernel_GBps": round(peak["kernel"], 3)},
        "roofline": None,
        "roofline_ring_copy": _ring_roofline(llama, measured_peak),
        "cpu_baseline": None if args.skip_cpu_baseline else cpu_llama_decode_baseline(),
    }
    gc.collect()
    torch.cuda.empty_cache()

    # ---- the same decode with each layer's attention and three MLP projections as separate units
    if not args.skip_finer_units:
        fine = bench_llama7b(args.budget_gb, args.prefill, args.steps, args.warmup, args.copy_engine,
                             include_patterns=FINER_UNITS, ring_order=args.ring_order)
        fine_check = fine.pop("_check")
        same = (torch.equal(fine_check["last_logits"], check["last_logits"])
                and torch.equal(fine_check["tokens"], check["tokens"]))
        line["llama7b_finer_units"] = {
            "include_patterns": list(FINER_UNITS),
            "streamed_units": fine["streamed_layers"], "resident_units": fine["resident_layers"],
            "streamed_bytes_per_token": fine["streamed_bytes_per_token"],
            "tok_s": round(fine["decode_tok_s"], 3), "ms_per_token": round(fine["ms_per_token"], 3),
            "decode_effective_GBps": round(fine["decode_effective_GBps"], 3),
            "pct_of_measured_peak": round(100 * fine["decode_effective_GBps"] / measured_peak, 2),
            "gpu_weight_bytes": fine["gpu_weight_bytes"],
            "copy_policy": fine["copy_policy"],
            "ring_order": fine["ring_order"],
            "ring_copies": _ring_roofline(fine, measured_peak),
            "prefill_logits_and_tokens_bitwise_equal_to_layer_units": same,
        }
        _log(f"llama7b finer units: {line['llama7b_finer_units']}")
        del fine, fine_check
        gc.collect()
        torch.cuda.empty_cache()
        if not same:
            print("bench: the finer-unit decode differs from the whole-layer decode", file=sys.stderr)
            return 1

    if not args.skip_encoded:
        enc = bench_llama7b(args.budget_gb, args.prefill, args.steps, args.warmup, args.copy_engine,
                            ring_order=args.ring_order, encode=True)
        enc_check = enc.pop("_check")
        same = (torch.equal(enc_check["last_logits"], check["last_logits"])
                and torch.equal(enc_check["tokens"], check["tokens"]))
        line["llama7b_encoded_blocks"] = _encoded_summary(enc, measured_peak, llama["decode_tok_s"])
        line["llama7b_encoded_blocks"]["prefill_logits_and_tokens_bitwise_equal_to_raw_blocks"] = same
        _log(f"llama7b encoded blocks: {line['llama7b_encoded_blocks']}")
        del enc, enc_check
        gc.collect()
        torch.cuda.empty_cache()
        if not same:
            print("bench: the decode with encoded blocks differs from the decode with raw blocks", file=sys.stderr)
            return 1
        # resident units also kept exponent-coded in HBM: more fit the budget, fewer stream. Attention and
        # MLP projections as separate units: smaller ring and decode slots leave more room for them.
        enc = bench_llama7b(args.budget_gb, args.prefill, args.steps, args.warmup, args.copy_engine,
                            include_patterns=FINER_UNITS, ring_order=args.ring_order, encode=True,
                            encode_resident=True)
        enc_check = enc.pop("_check")
        same = (torch.equal(enc_check["last_logits"], check["last_logits"])
                and torch.equal(enc_check["tokens"], check["tokens"]))
        line["llama7b_encoded_resident"] = _encoded_summary(enc, measured_peak, llama["decode_tok_s"])
        line["llama7b_encoded_resident"]["prefill_logits_and_tokens_bitwise_equal_to_raw_blocks"] = same
        line["llama7b_encoded_resident"]["include_patterns"] = list(FINER_UNITS)
        _log(f"llama7b encoded resident: {line['llama7b_encoded_resident']}")
        del enc, enc_check
        gc.collect()
        torch.cuda.empty_cache()
        if not same:
            print("bench: the decode with layers encoded in HBM differs from the decode with raw blocks",
                  file=sys.stderr)
            return 1

    # ---- the scatter microbenchmark and the scatter kernel's HBM roofline
    if not args.skip_scatter:
        res = bench_scatter(args.scatter_steps, 1, args.chunk_mib, args.tensors, args.copy_engine,
                            verify=not args.skip_verify)
        _log(f"scatter workload: {res['effective_GBps']:.2f} GB/s effective, link {res['link_GBps']:.2f} GB/s, "
             f"scatter kernel {res['scatter_hbm_GBps']:.0f} GB/s HBM, mismatches {res['mismatched_tensors']}")
        if res["mismatched_tensors"]:
            print(f"bench: {res['mismatched_tensors']} destination tensors differ from the streamed bytes",
                  file=sys.stderr)
            return 1
        line["roofline"] = {"kernel": "scatter_kernel", "bound": "hbm", "achieved": round(res["scatter_hbm_GBps"], 1),
                            "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                            "frac": round(res["scatter_hbm_GBps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                            "avg_launch_ms": round(res["scatter_avg_ms"], 4),
                            "algorithmic_bytes_per_launch": int(res["scatter_bytes_per_launch"]),
                            "workload": "scatter microbenchmark (the placement of every tensor outside the ring)"}
        copy = device_copy_probe(args.chunk_mib * MiB)
        line["roofline"]["device_copy_GBps"] = copy["GBps"]
        line["roofline"]["frac_of_device_copy"] = round(res["scatter_hbm_GBps"] / copy["GBps"], 4)
        line["scatter"] = {
            "workload": "2000 bf16 tensors, log-uniform 4 KiB-64 MiB, seed 1, "
                        f"{args.chunk_mib} MiB pinned chunks, 2-slot ring, one scatter launch per chunk",
            "payload_bytes": res["payload_bytes"], "chunks": res["n_chunks"], "steps": args.scatter_steps,
            "ms_per_step": round(res["ms_per_step"], 3), "effective_GBps": round(res["effective_GBps"], 3),
            "link_GBps": round(res["link_GBps"], 3),
            "pct_of_measured_peak": round(100 * res["link_GBps"] / measured_peak, 2),
            "cpu_baseline": None if args.skip_cpu_baseline else cpu_baseline_scatter(res["chunks"]),
        }
        del res
        gc.collect()
        torch.cuda.empty_cache()
        if not args.no_traffic:
            tr = measure_traffic(args)
            if tr is not None:
                line["roofline"]["traffic"] = int(tr["traffic"])
                line["roofline"]["traffic_detail"] = {k: (int(v) if "bytes" in k else v) for k, v in tr.items()
                                                      if k not in ("traffic", "ring_copy", "expcode_decode")}
                _log(f"traffic per scatter launch: {tr['traffic'] / 1e9:.3f} GB "
                     f"(algorithmic {line['roofline']['algorithmic_bytes_per_launch'] / 1e9:.3f} GB)")
                ring_tr = tr.get("ring_copy")
                if ring_tr is not None and line.get("roofline_ring_copy"):
                    # HBM bytes: the writes; the reads come from host memory over the link
                    line["roofline_ring_copy"]["traffic"] = int(ring_tr["hbm_write_bytes_per_launch"])
                    line["roofline_ring_copy"]["traffic_detail"] = {k: int(v) for k, v in ring_tr.items()}
                    _log(f"traffic per ring copy: {ring_tr}")
                dec_tr = tr.get("expcode_decode")
                enc_roof = (line.get("llama7b_encoded_blocks") or {}).get("ring_copies")
                if dec_tr is not None and enc_roof:
                    enc_roof["traffic"] = int(dec_tr["hbm_write_bytes_per_launch"])
                    enc_roof["traffic_detail"] = {k: int(v) for k, v in dec_tr.items() if v is not None}
                    _log(f"traffic per encoded-block decode: {dec_tr}")
    if not args.skip_mlp:
        gc.collect()
        torch.cuda.empty_cache()
        line["mlp8"] = bench_mlp(20, args.copy_engine, ring_order=args.ring_order)
        _log(f"mlp8: {line['mlp8']}")
        if not line["mlp8"]["bitwise_equal_to_resident"]:
            print("bench: the streamed MLP forward differs from the resident forward", file=sys.stderr)
            return 1
        if not args.skip_encoded:
            gc.collect()
            torch.cuda.empty_cache()
            enc = bench_mlp(20, args.copy_engine, ring_order=args.ring_order, encode=True)
            enc["link_bytes_ratio"] = round(enc["link_bytes_per_forward"] / enc["streamed_bytes_per_forward"], 4)
            enc["eager_speedup_vs_raw_blocks"] = round(line["mlp8"]["eager_ms_per_forward"]
                                                       / enc["eager_ms_per_forward"], 4)
            line["mlp8"]["encoded_blocks"] = enc
            _log(f"mlp8 encoded blocks: {enc}")
            if not enc["bitwise_equal_to_resident"]:
                print("bench: the streamed MLP forward with encoded blocks differs from the resident forward",
                      file=sys.stderr)
                return 1
    if not args.skip_dit:
        gc.collect()
        torch.cuda.empty_cache()
        line["dit"] = bench_dit(12.0, args.dit_tokens, 512, args.dit_steps)
        _log(f"dit: {line['dit']}")
        if not line["dit"]["bitwise_equal_to_resident"]:
            print("bench: the streamed DiT step differs from the resident step", file=sys.stderr)
            return 1
    if not args.skip_70b:
        gc.collect()
        torch.cuda.empty_cache()
        line["fp8_linear"] = bench_fp8_linear()
        _log(f"fp8 linear: {line['fp8_linear']}")
        line["fp8_prefill"] = bench_fp8_prefill()
        _log(f"fp8 prefill: {line['fp8_prefill']}")
        line["llama70b_fp8"] = bench_llama70b_fp8(24.0, 8, 64, 8, args.layers_70b, ring_order=args.ring_order)
        if not args.skip_cpu_baseline and "skipped" not in line["llama70b_fp8"]:
            line["llama70b_fp8"]["cpu_baseline"] = cpu_llama70b_decode_baseline()
        _log(f"70b: {line['llama70b_fp8']}")
    print(json.dumps(line), flush=True)
    return 0


def _finish() -> None:
    """Leave nothing in flight at exit: drop what the legs left for the collector (their managers are already
    released), wait for the device, and let the library release its own threads, staging buffers, streams
    and events (``ftx_shutdown``) while the runtime is still up."""
    import gc

    gc.collect()
    if "torch" in sys.modules:
        import torch

        if torch.cuda.is_available() and torch.cuda.is_initialized():
            torch.cuda.synchronize()
    nat = sys.modules.get("flextensor_amd._native")
    if nat is not None and nat.live():
        nat.shutdown()


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    try:
        code = main()
    finally:
        _finish()
    sys.exit(code)
