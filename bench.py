"""Benchmark: Qwen3-Omni-thinker-shaped paged decode on one MI355X (BASELINE config c3).

One step = one pass of the attention hot path for one layer over the whole
ragged batch, through the drop-in surface M*'s engine calls:

  BatchedCacheManager.plan_attention([1]*B)  host FIFO allocation of new pages,
                                             block-table delta, mi_pack, mi_decode_plan
  BatchedCacheManager.run_attention(q, k, v) mi_kv_append, decode kernel, merge kernel
  advance_seq_lens()

Inputs are resident in HBM before timing: a 262144-page bf16 KV pool
(8.6 GB, random N(0,1)), B=256 requests with log-uniform [512, 32768]
contexts on randomly permuted pages (seed 2).  ``value`` = decode tokens/s
= B / wall-clock ms per step.  ``roofline`` reports the decode kernel alone:
algorithmic bytes of one launch (KV read of every token + q read + o write +
index arrays; split-KV partials excluded) over its average duration from HIP
events on the launch stream.  ``cpu_baseline`` times the CPU restatement
(``oracle/``) on a bounded sample of the same requests on the host cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from mstar_amd import _lib  # noqa: E402
from mstar_amd import synthetic as S  # noqa: E402
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager  # noqa: E402
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per decode launch measured by rocprofv3 --pmc (FETCH_SIZE and
# WRITE_SIZE passes scaled by a copy-kernel calibration); the summary that
# holds the figure is regenerated whenever the decode kernel changes.
TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "decode_kernel_{config}_pmc.md")
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged decode attn tokens/s + achieved HBM GB/s (% peak), 1 MI355X, B=256"


def measured_traffic(config: str) -> tuple[int | None, int | None]:
    """(``traffic_bytes_per_launch``, ``algorithmic_bytes_per_launch``) from the
    committed rocprofv3 --pmc summary of ``config``, or (None, None)."""
    vals = {}
    try:
        with open(TRAFFIC_PROFILE.format(config=config)) as f:
            for line in f:
                for key in ("traffic_bytes_per_launch", "algorithmic_bytes_per_launch"):
                    if line.startswith(key + ":"):
                        vals[key] = int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return vals.get("traffic_bytes_per_launch"), vals.get("algorithmic_bytes_per_launch")


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def fill_pool(kv: torch.Tensor, spec, device: torch.device):
    """N(0,1) K/V drawn in bf16 from a seeded device generator, every layer.

    An fp8 pool is quantised per (layer, K|V, kv-head) with s = amax/448 over
    the layer (two passes over the same draws); returns the fp32 scales
    ``[layers, 2, num_kv_heads]`` or None for a bf16 pool.
    """
    gen = torch.Generator(device=device).manual_seed(spec.seed)
    chunk = 1 << 14
    pages = kv.shape[1]
    if kv.dtype != torch.float8_e4m3fn:
        for layer in range(kv.shape[0]):
            for p0 in range(0, pages, chunk):
                kv[layer, p0:p0 + chunk].normal_(generator=gen)
        return None
    tmp = torch.empty((chunk,) + tuple(kv.shape[2:]), dtype=torch.bfloat16, device=device)
    all_scales = []
    for layer in range(kv.shape[0]):
        amax = torch.zeros(2, spec.num_kv_heads, device=device)
        state = gen.get_state()
        for p0 in range(0, pages, chunk):
            t = tmp[:min(chunk, pages - p0)].normal_(generator=gen)
            amax = torch.maximum(amax, t.abs().amax(dim=(0, 2, 4)).float())
        scales = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
        inv = (1.0 / scales).view(1, 2, 1, spec.num_kv_heads, 1)
        gen.set_state(state)
        for p0 in range(0, pages, chunk):
            n = min(chunk, pages - p0)
            t = tmp[:n].normal_(generator=gen)
            kv[layer, p0:p0 + n] = (t.float() * inv).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        all_scales.append(scales)
    return torch.stack(all_scales).contiguous()


# Layers of the pool a decode bench cycles through: one per step, as a
# model's layer-steps would.  A working set below the 256 MB MALL (c1, and
# c2 at 323 MB) would otherwise be served partly from the MALL when the same
# layer is read step after step; three layers put about 1 GB between two
# reads of the same pages.
MALL_BYTES = 256 << 20


def decode_layers(bt) -> int:
    s = bt.spec
    elem = 1 if s.kv_dtype == "fp8" else 2
    working = bt.total_kv_tokens * s.num_kv_heads * s.head_dim * 2 * elem
    return 3 if working < 4 * MALL_BYTES else 1


def setup(spec_name: str, device: torch.device, layers: int | None = None, trace_ranges: bool = False):
    bt = S.make_batch(spec_name)
    s = bt.spec
    b = len(bt.kv_len)
    if layers is None:
        layers = decode_layers(bt)
    cfg = KVCacheConfig(num_layers=layers, num_kv_heads=s.num_kv_heads, head_dim=s.head_dim,
                        max_seq_len=40960, max_num_pages=s.pool_pages, page_size=s.page_size,
                        num_qo_heads=s.num_qo_heads)
    kv_dtype = torch.float8_e4m3fn if s.kv_dtype == "fp8" else torch.bfloat16
    kv = torch.empty(layers, s.pool_pages, 2, s.page_size, s.num_kv_heads, s.head_dim, dtype=kv_dtype,
                     device=device)
    scales = fill_pool(kv, s, device)
    mgr = PagedAllocationManager(cfg, kv, device=device)
    # Steady state: each request already holds its T-1 cached tokens on the
    # drawn (random) pages; the allocator's free list holds the rest of the
    # permutation, so new pages keep coming from random places.
    used = set(bt.kv_indices.tolist())
    perm_rest = [p for p in torch.randperm(s.pool_pages, generator=torch.Generator().manual_seed(s.seed + 100)).tolist()
                 if p not in used]
    mgr.page_allocator.free_pages.clear()
    mgr.page_allocator.free_pages.extend(perm_rest)
    rids = [f"req{i}" for i in range(b)]
    for i, r in enumerate(rids):
        mgr.add_request(r, ["main"])
        st = mgr.get_state(r, "main")
        st.page_indices = bt.kv_indices[bt.kv_indptr[i]:bt.kv_indptr[i + 1]].tolist()
        st.seq_len = int(bt.kv_len[i]) - 1
        st.position_id_start = st.seq_len
    bufs = WorkspaceBufferManager(512 << 20, device)  # the reference's per-label workspace size
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, device, kv_scales=scales,
                             enable_nvtx=trace_ranges)
    g = torch.Generator().manual_seed(s.seed + 1)
    q = torch.randn(b, s.num_qo_heads, s.head_dim, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(b, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(b, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(device)
    return bt, cfg, kv, mgr, cm, rids, q, k, v


def decode_bytes(seq_lens_after: np.ndarray, total_pages: int, s) -> int:
    """Algorithmic HBM bytes of one decode-kernel launch (partials excluded)."""
    b = len(seq_lens_after)
    elem = 1 if s.kv_dtype == "fp8" else 2
    kv = int(seq_lens_after.sum()) * s.num_kv_heads * s.head_dim * 2 * elem
    qo = b * s.num_qo_heads * s.head_dim * 2 * 2
    idx = 4 * (total_pages + 3 * b)
    scales = 2 * s.num_kv_heads * 4 if elem == 1 else 0
    return kv + qo + idx + scales


def _layer_scales(cm, layer: int = 0):
    if cm.kv_scales is None:
        return None, None
    return cm.kv_scales[layer, 0], cm.kv_scales[layer, 1]


def step_once(cm, q, k, v, b, events=None, layer: int = 0):
    """One layer-step: plan (pack + split-KV plan), append, decode + merge, advance."""
    cm.plan_attention([1] * b)
    wrapper = cm._plan_states["main"].wrapper
    kv_layer = cm.kv_cache[layer]
    ks, vs = _layer_scales(cm, layer)
    wrapper.set_kv_cache(kv_layer, k, v, k_scale=ks, v_scale=vs)
    if events is None:
        out = wrapper.run(q, kv_layer, k_scale=ks, v_scale=vs)
    else:
        out = _run_split(wrapper, q, kv_layer, ks, vs, events)
    cm.advance_seq_lens()
    return out


def _decode_args(w, q, kv_layer, ks, vs, out):
    desc = _lib.paged_kv_desc(kv_layer, ks, vs)
    return (q.data_ptr(), _lib.MI_BF16, q.stride(0), q.stride(1), desc, None, w._indptr.data_ptr(),
            w._indices.data_ptr(), w._last.data_ptr(), w._n_req, w.num_qo_heads, 0, 1.0 / math.sqrt(w.head_dim),
            w._workspace.data_ptr(), w._workspace.numel(), out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_ptr(q.device))


def _run_split(w, q, kv_layer, ks, vs, events):
    """wrapper.run() as its two C entry points, with HIP events around the decode kernel."""
    out = torch.empty_like(q)
    args = _decode_args(w, q, kv_layer, ks, vs, out)
    e0, e1, e2 = events
    e0.record()
    _lib.check(_lib.lib().mi_decode_attend(*args), "mi_decode_attend")
    e1.record()
    _lib.check(_lib.lib().mi_decode_merge(*args), "mi_decode_merge")
    e2.record()
    return out


def decode_graph_us(cm, q, steps: int, per_graph: int = 12) -> tuple[float, float]:
    """(decode kernel us, decode + merge us) per launch of the current plan, from
    HIP graph replays: at least ``per_graph`` launches (the same number on every
    layer of the pool, in turn) captured into one graph; HIP events around each
    replay on the launch stream.  Replays time the GPU alone, without the host
    issue gaps that sit between a short kernel and the events around it; the
    graph launch itself is spread over the launches of one replay."""
    w = cm._plan_states["main"].wrapper
    layers = cm.kv_cache.shape[0]
    per_layer = -(-per_graph // layers)
    out = torch.empty_like(q)
    argv = [_decode_args(w, q, cm.kv_cache[i], *_layer_scales(cm, i), out) for i in range(layers)]
    L = _lib.lib()
    n = per_layer * layers

    def attend():
        for i in range(n):
            _lib.check(L.mi_decode_attend(*argv[i % layers][:-1], _lib.stream_ptr(q.device)), "mi_decode_attend")

    def both():
        for i in range(n):
            a = (*argv[i % layers][:-1], _lib.stream_ptr(q.device))
            _lib.check(L.mi_decode_attend(*a), "mi_decode_attend")
            _lib.check(L.mi_decode_merge(*a), "mi_decode_merge")

    return (_graph_us(attend, q.device, steps, per_graph=1) / n, _graph_us(both, q.device, steps, per_graph=1) / n)


def host_cpu() -> dict:
    """The host's CPU as /proc/cpuinfo names it, and its logical CPU count."""
    info = {"model": "", "family": "", "model_number": "", "stepping": "", "logical_cpus": os.cpu_count()}
    keys = {"model name": "model", "cpu family": "family", "model": "model_number", "stepping": "stepping"}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if info["model"]:
                        break  # first processor block read
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                if k in keys and not info[keys[k]]:
                    info[keys[k]] = v
    except OSError:
        pass
    return info


def cpu_baseline(bt, kv_gpu, q, k, v, scales=None, budget_s: float = 20.0, min_runs: int = 2):
    """The CPU restatement (oracle/) of one whole step of the batch: FIFO pack, append,
    fp32 paged attention, on the host threads this process is given.

    Runs the whole batch until ``budget_s`` has passed and at least
    ``min_runs`` runs are done; reports the median.  Layer 0 of the pool, the
    batch's pages only (copied to host memory once, outside the timing)."""
    from oracle import attention as A
    from oracle import packing as P

    s = bt.spec
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    nreq = len(bt.kv_len)
    pages = bt.kv_indices
    uniq = np.unique(pages)
    remap = np.zeros(s.pool_pages, dtype=np.int64)
    remap[uniq] = np.arange(len(uniq))
    cache = kv_gpu[0, torch.as_tensor(uniq, device=kv_gpu.device)].cpu()
    idx = remap[pages].astype(np.int32)
    qc, kc, vc = q[:nreq].cpu(), k[:nreq].cpu(), v[:nreq].cpu()
    ks = vs = None
    if scales is not None:
        ks, vs = scales[0, 0].cpu(), scales[0, 1].cpu()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        states, extra = [], []
        for i in range(nreq):
            pl = idx[bt.kv_indptr[i]:bt.kv_indptr[i + 1]].tolist()
            cached = int(bt.kv_len[i]) - 1
            keep = -(-cached // s.page_size)
            states.append(P.ReqState(pages=pl[:keep], seq_len=cached))
            extra += pl[keep:]  # a page the new token opens comes from the free list
        pool = P.FifoPages(0)
        pool.free.extend(extra)
        packed = P.pack(states, [1] * nreq, pool, s.page_size)
        loc = packed.kv_locations
        A.append(cache, loc[:, 0], loc[:, 1], kc, vc, ks, vs)
        A.paged_attention(qc, cache, None, packed.kv_indptr, packed.kv_indices, packed.last_page_len, causal=False,
                          k_scale=ks, v_scale=vs)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cpu = host_cpu()
    return {
        "value": nreq / med,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "ms_per_step": med * 1e3,
        "host_logical_cpus": cpu["logical_cpus"],
        "cpu_model": cpu["model"],
        "cpu_family_model_stepping": f"{cpu['family']}/{cpu['model_number']}/{cpu['stepping']}",
        "sample": (f"the whole {s.name} step: {nreq} requests, {int(bt.kv_len.sum())} KV tokens; FIFO pack + append "
                   f"+ fp32 paged attention (oracle/), median of {len(times)} runs, {torch.get_num_threads()} host "
                   f"threads (this process's share of the box's {cpu['logical_cpus']} logical CPUs), "
                   f"CPU: {cpu['model']}"),
    }


def copy_calibration(dev) -> int:
    """A plain copy of 1 GiB, three times: 1 GiB read + 1 GiB written per launch."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    for i in range(3):
        dst.copy_(src)
        ev[i + 1].record()
    torch.cuda.synchronize()
    ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(3)]
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "ms": ms,
                      "copy_GBps_read_plus_write": [2 * n / (m * 1e-3) / 1e9 for m in ms]}), flush=True)
    return 0


WORKLOADS = {
    "c1": "c1: CPU-baseline decode shape (B=8, 8 q / 2 kv heads), one layer-step of pack+plan+append+decode+merge",
    "c2": "c2: Orpheus (Llama-3.2-3B) decode, one layer-step of pack+plan+append+decode+merge",
    "c3": "c3: Qwen3-Omni thinker decode, one layer-step of pack+plan+append+decode+merge",
    "c4": "c4: BAGEL (Qwen2.5-7B) ragged chunked prefill + decode mix, one layer-step of plan+append+attention",
    "c5": "c5: Qwen3-Omni thinker decode on an fp8-e4m3 KV cache, one layer-step of pack+plan+append+decode+merge",
}


def hbm_read_ceiling(buf: torch.Tensor, steps: int = 10, nbytes: int | None = None) -> dict:
    """The box's plain read rate over ``buf`` (the KV pool layer the decode
    kernel streams): ``mi_hbm_read`` with the decode kernel's 16-byte
    non-temporal loads, median of ``steps`` launches timed with HIP events.
    With ``nbytes`` (a job's size), each launch reads that many bytes, in turn
    from up to three disjoint regions of ``buf``, as the decode bench cycles
    pool layers, so a small job's ceiling is not served from the 256 MB
    Infinity Cache and carries the same launch ramp and tail."""
    dev = buf.device
    total = buf.numel() * buf.element_size() // 16 * 16
    size = total if nbytes is None else min(int(nbytes) // 16 * 16, total)
    regions = max(1, min(3, total // size))
    grid = 8 * torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(4 * grid, dtype=torch.int32, device=dev)
    stream = _lib.stream_ptr(dev)
    launch = lambda i: _lib.check(_lib.lib().mi_hbm_read(buf.data_ptr() + (i % regions) * size, size, sink.data_ptr(),
                                                         grid, stream), "mi_hbm_read")
    for i in range(regions):
        launch(i)
    evs = _kernel_events(steps, 2)
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        launch(i)
        e1.record()
    torch.cuda.synchronize()
    us = float(np.median([e0.elapsed_time(e1) for e0, e1 in evs])) * 1e3
    what = ("plain 16-byte non-temporal read of the KV pool layer" if nbytes is None else
            f"plain 16-byte non-temporal read of the job's size, {regions} region(s) of the pool layer in turn")
    return {"kernel": "hbm_read_kernel", "what": what, "bytes": size, "regions": regions, "us_median": us,
            "GBps": size / (us * 1e-6) / 1e9}


def _kernel_events(n: int, k: int):
    return [tuple(torch.cuda.Event(enable_timing=True) for _ in range(k)) for _ in range(n)]


def bench_decode(args, dev) -> dict:
    _log(f"setup {args.config} ...")
    bt, cfg, kv, mgr, cm, rids, q, k, v = setup(args.config, dev, trace_ranges=args.trace_ranges)
    s = bt.spec
    b = len(rids)
    layers = kv.shape[0]
    torch.cuda.synchronize()
    _log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        step_once(cm, q, k, v, b, layer=i % layers)
    torch.cuda.synchronize()

    # timed region 1: the full hot path per step, wall clock
    _log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step_once(cm, q, k, v, b, layer=i % layers)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps

    # timed region 2: same steps, decode and merge kernels bracketed by HIP events
    evs = _kernel_events(args.steps, 3)
    bytes_per = []
    for i in range(args.steps):
        seq_after = np.array([cm._get_state(r).seq_len + 1 for r in rids])
        step_once(cm, q, k, v, b, events=evs[i], layer=i % layers)
        bytes_per.append(decode_bytes(seq_after, sum(len(cm._get_state(r).page_indices) for r in rids), s))
    torch.cuda.synchronize()
    dec_ms = np.array([e0.elapsed_time(e1) for e0, e1, _ in evs])
    dm_ms = np.array([e0.elapsed_time(e2) for e0, _, e2 in evs])

    # timed region 3: the last step's plan, decode (and merge) launches replayed from a HIP graph
    seq_now = np.array([cm._get_state(r).seq_len for r in rids])
    graph_bytes = decode_bytes(seq_now, sum(len(cm._get_state(r).page_indices) for r in rids), s)
    dec_us, dm_us = decode_graph_us(cm, q, args.steps)
    achieved = graph_bytes / (dec_us * 1e-6) / 1e9
    kv_tokens = int(seq_now.sum())
    ceiling = hbm_read_ceiling(kv[0])
    ceiling_job = hbm_read_ceiling(kv[0], nbytes=graph_bytes)
    lo, hi = s.ctx[1], s.ctx[2]
    traffic, traffic_alg = measured_traffic(s.name)
    res = {
        "metric": METRIC if s.name == "c3" else f"paged decode attn tokens/s + achieved HBM GB/s, 1 MI355X, B={b}",
        "value": b / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 KV, bf16 q/o, fp32 accumulate" if s.kv_dtype == "fp8" else "bf16",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[s.name],
            "batch": b, "num_qo_heads": s.num_qo_heads, "num_kv_heads": s.num_kv_heads, "head_dim": s.head_dim,
            "page_size": s.page_size, "context": f"{s.ctx[0]} [{lo}, {hi}]", "kv_pool_pages": s.pool_pages,
            "kv_layers_cycled": layers, "kv_dtype": s.kv_dtype, "kv_tokens_at_end": kv_tokens,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes over the {s.name} bench, scaled by a "
                               f"1 GiB copy; per decode launch of a plan with {traffic_alg} algorithmic bytes"
                               if traffic is not None else None),
            "traffic_per_algorithmic_byte": traffic / traffic_alg if traffic and traffic_alg else None,
            "kernel": "decode_kernel",
            "kernel_us": dec_us,
            "kernel_us_how": (f"HIP graph replay of {-(-12 // layers) * layers} decode launches of the last step's plan "
                              f"({layers} pool layer(s) in turn), HIP events on the launch stream"),
            "algorithmic_bytes": graph_bytes,
            "decode_plus_merge_us": dm_us,
            "kernel_us_events_in_step_loop": float(dec_ms.mean()) * 1e3,
            "decode_plus_merge_us_events_in_step_loop": float(dm_ms.mean()) * 1e3,
            "algorithmic_bytes_step_loop_mean": int(np.mean(bytes_per)),
            "hbm_read_ceiling": ceiling,
            "frac_of_read_ceiling": achieved / ceiling["GBps"],
            "hbm_read_same_bytes": ceiling_job,
            "frac_of_same_bytes_read": ceiling_job["us_median"] / dec_us,
        },
    }
    pos_now = seq_now
    if not args.no_extra:
        res["rope"] = bench_rope(q, k, pos_now, args.steps)
        res["rope_append"] = bench_rope_append(cm, q, k, v, pos_now, args.steps)
        res["kv_transfer"] = bench_transfer(kv, args.steps)
        res["decode_side"] = bench_decode_side(dev, args.steps)
    if not args.no_cpu_baseline:
        _log("cpu baseline ...")
        res["cpu_baseline"] = cpu_baseline(bt, kv, q, k, v, cm.kv_scales, min_runs=10 if s.name == "c1" else 2)
    return res


def _graph_us(fn, device, steps: int, per_graph: int = 20) -> float:
    """Mean time of one ``fn()`` from HIP graph replays of ``per_graph`` captured calls.

    The kernels involved are shorter than a Python launch, so host-issued
    launches would time the host; replaying a captured graph times the GPU.
    """
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    evs = _kernel_events(max(steps // 5, 3), 2)
    for e0, e1 in evs:
        e0.record()
        graph.replay()
        e1.record()
    torch.cuda.synchronize()
    return float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e3 / per_graph


def bench_rope(q, k, positions: np.ndarray, steps: int, per_graph: int = 20) -> dict:
    """apply_rope on this step's q and k (in place, on copies): HBM read + write of both."""
    from mstar_amd.rope import apply_rope_pos_ids_inplace

    qc, kc = q.clone(), k.clone()
    pos = torch.as_tensor(positions, dtype=torch.int64, device=q.device)
    us = _graph_us(lambda: apply_rope_pos_ids_inplace(qc, kc, pos, rope_theta=1e6), q.device, steps, per_graph)
    nbytes = 2 * (qc.numel() + kc.numel()) * qc.element_size() + pos.numel() * 8
    return {"kernel": "rope_kernel", "what": "apply_rope_pos_ids_inplace on the step's q [B, Hq, D] and k [B, Hkv, D], "
            f"{per_graph} launches per HIP graph replay", "kernel_us": us, "algorithmic_bytes": nbytes,
            "GBps": nbytes / (us * 1e-6) / 1e9}


def bench_rope_append(cm, q, k, v, positions: np.ndarray, steps: int, per_graph: int = 20) -> dict:
    """One layer's RoPE + K/V append: two launches (rope_kernel, append_kernel) vs rope_append_kernel.

    Both write this step's slots of layer 0 (the decode wrapper's planned
    locations); q and k are copies rotated in place.
    """
    from mstar_amd.rope import apply_rope_pos_ids_inplace

    w = cm._plan_states["main"].wrapper
    layer = cm.kv_cache[0]
    ks, vs = _layer_scales(cm)
    qc, kc = q.clone(), k.clone()
    pos = torch.as_tensor(positions, dtype=torch.int64, device=q.device)

    def two():
        apply_rope_pos_ids_inplace(qc, kc, pos, rope_theta=1e6)
        w.set_kv_cache(layer, kc, v, k_scale=ks, v_scale=vs)

    def one():
        w.rope_set_kv_cache(layer, qc, kc, v, pos, rope_theta=1e6, k_scale=ks, v_scale=vs)

    t_two = _graph_us(two, q.device, steps, per_graph)
    t_one = _graph_us(one, q.device, steps, per_graph)
    kv_elem = layer.element_size()
    # fused: read q, k, v and positions, write q, k and the cache's K and V rows
    nbytes = (2 * q.numel() + 2 * k.numel() + v.numel()) * q.element_size() + pos.numel() * 8 \
        + 2 * k.numel() * kv_elem + 16 * q.shape[0]
    return {"kernel": "rope_append_kernel", "what": "decode wrapper rope_set_kv_cache vs apply_rope_pos_ids_inplace + "
            f"set_kv_cache on the step's q, k, v, {per_graph} per HIP graph replay",
            "two_launches_us": t_two, "fused_us": t_one, "algorithmic_bytes": nbytes,
            "GBps": nbytes / (t_one * 1e-6) / 1e9}


def bench_transfer(kv_layer: torch.Tensor, steps: int, pages: int = 32768, host_pages: int = 4096) -> dict:
    """KV page transfer at the workload's page shape ``[2, ps, Hkv, D]``, one layer.

    * ``mi_kv_copy_tokens``: ``pages`` whole pages from one pool to another,
      random page ids on both sides (remote read / snapshot); HBM read + write;
    * ``mi_kv_wire_pack``: the same pages into a contiguous wire buffer;
    * ``mi_kv_copy_tokens`` into a pinned host pool (CPU offload), ``host_pages``
      pages, bounded by the host link rather than HBM.
    Records are uploaded before the timed launches; HIP events bracket
    ``max(steps // 5, 5)`` launches each on the current stream.
    """
    import ctypes

    from mstar_amd import _lib
    from mstar_amd import kv_transfer as KT

    if kv_layer.dim() == 6:  # [layers, pages, 2, ps, Hkv, D]
        kv_layer = kv_layer[0]
    dev = kv_layer.device
    shape = (1, pages) + tuple(kv_layer.shape[1:])
    bits = torch.uint8 if kv_layer.element_size() == 1 else torch.int16
    src = torch.empty(shape, dtype=bits, device=dev)
    src.random_(0, 127)
    dst = torch.empty_like(src)
    src, dst = src.view(kv_layer.dtype), dst.view(kv_layer.dtype)
    host = torch.empty((1, host_pages) + tuple(kv_layer.shape[1:]), dtype=kv_layer.dtype, pin_memory=True)
    g = torch.Generator().manual_seed(0)
    rec = torch.stack([torch.randperm(pages, generator=g), torch.randperm(pages, generator=g)]).to(torch.int32).to(dev)
    hrec = torch.arange(host_pages, dtype=torch.int32, device=dev)
    page_bytes = src[0, 0].numel() * src.element_size()
    wire = torch.empty(pages * page_bytes, dtype=torch.uint8, device=dev)
    sd, dd, hd = KT.pool_desc(src), KT.pool_desc(dst), KT.pool_desc(host)
    L = _lib.lib()
    st = _lib.stream_ptr(dev)
    d0, s0 = rec.data_ptr(), rec.data_ptr() + 4 * pages

    def copy():
        return L.mi_kv_copy_tokens(ctypes.byref(sd), ctypes.byref(dd), s0, d0, None, None, pages, 0, 1, st)

    def pack():
        return L.mi_kv_wire_pack(ctypes.byref(sd), s0, None, None, None, pages, 0, 1, wire.data_ptr(), wire.numel(), st)

    def offload():
        return L.mi_kv_copy_tokens(ctypes.byref(sd), ctypes.byref(hd), s0, hrec.data_ptr(), None, None, host_pages,
                                   0, 1, st)

    def device_copy():  # contiguous torch copy of the same bytes: what a plain HBM copy reaches
        dst.view(-1).copy_(src.view(-1))
        return 0

    n = max(steps // 5, 5)
    out = {"kernel": "kv_segments_kernel", "page_bytes": page_bytes,
           "what": f"{pages} random whole pages pool->pool and pool->wire, {host_pages} pages pool->pinned host; "
                   "torch_contiguous_copy = dst.copy_(src) of the same bytes, for scale"}
    for name, fn, moved, count_both in (("copy", copy, pages * page_bytes, True),
                                        ("wire_pack", pack, pages * page_bytes, True),
                                        ("offload_to_host", offload, host_pages * page_bytes, False),
                                        ("torch_contiguous_copy", device_copy, pages * page_bytes, True)):
        for _ in range(3):
            _lib.check(fn(), name)
        evs = _kernel_events(n, 2)
        for e0, e1 in evs:
            e0.record()
            _lib.check(fn(), name)
            e1.record()
        torch.cuda.synchronize()
        us = float(np.median([a.elapsed_time(b) for a, b in evs])) * 1e3
        nbytes = moved * (2 if count_both else 1)
        out[name] = {"kernel_us_median": us, "algorithmic_bytes": nbytes, "GBps": nbytes / (us * 1e-6) / 1e9}
        if count_both:
            out[name]["hbm_frac"] = out[name]["GBps"] / HBM_PEAK_GBS
    return out


def _side_decode(dev, steps: int, hq: int, hkv: int, d: int, lens: np.ndarray, dtype: torch.dtype, seed: int,
                 pool_pages: int | None = None) -> dict:
    """Decode kernel time per launch (HIP graph replays of 4 launches of one plan) for
    one batch of contexts ``lens`` on random pages, page 16, the given dtype."""
    from mstar_amd.paged_attention import PagedDecodeWrapper

    ps, b = 16, len(lens)
    g = torch.Generator().manual_seed(seed)
    pages = (lens + ps - 1) // ps
    pool = pool_pages or int(pages.sum()) + 64
    perm = torch.randperm(pool, generator=g).numpy().astype(np.int32)
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    kv_indices = perm[: kv_indptr[-1]]
    last = (lens - (pages - 1) * ps).astype(np.int32)
    cache = torch.empty(pool, 2, ps, hkv, d, dtype=dtype, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    for p0 in range(0, pool, 1 << 14):
        cache[p0:p0 + (1 << 14)].normal_(generator=gen)
    q = torch.randn(b, hq, d, device=dev).to(dtype)
    w = PagedDecodeWrapper(torch.empty(512 << 20, dtype=torch.uint8, device=dev), hq, hkv, d, ps, device=dev)
    w.plan(torch.from_numpy(kv_indptr), torch.from_numpy(kv_indices), torch.from_numpy(last), dtype=dtype)
    out = torch.empty_like(q)
    args = (q.data_ptr(), _lib.TORCH_TO_MI[dtype], q.stride(0), q.stride(1), _lib.paged_kv_desc(cache), None,
            w._indptr.data_ptr(), w._indices.data_ptr(), w._last.data_ptr(), b, hq, 0, 1.0 / math.sqrt(d),
            w._workspace.data_ptr(), w._workspace.numel(), out.data_ptr(), out.stride(0), out.stride(1))
    L = _lib.lib()

    def attend():
        for _ in range(4):
            _lib.check(L.mi_decode_attend(*args, _lib.stream_ptr(dev)), "mi_decode_attend")

    def both():
        for _ in range(4):
            _lib.check(L.mi_decode_attend(*args, _lib.stream_ptr(dev)), "mi_decode_attend")
            _lib.check(L.mi_decode_merge(*args, _lib.stream_ptr(dev)), "mi_decode_merge")

    us = _graph_us(attend, dev, steps, per_graph=1) / 4
    us_dm = _graph_us(both, dev, steps, per_graph=1) / 4
    esz = cache.element_size()
    nbytes = int(lens.sum()) * hkv * d * 2 * esz + b * hq * d * q.element_size() * 2 + 4 * (int(pages.sum()) + 3 * b)
    del cache
    return {"batch": b, "heads": f"{hq} q / {hkv} kv", "head_dim": d, "kv_dtype": str(dtype).replace("torch.", ""),
            "kv_tokens": int(lens.sum()), "kernel_us": us, "decode_plus_merge_us": us_dm, "algorithmic_bytes": nbytes,
            "GBps": nbytes / (us * 1e-6) / 1e9, "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_decode_side(dev, steps: int) -> dict:
    """Decode at head_dim 256 and over fp32 pools, beside the configuration's step.

    * ``d256_c3_bytes``: the c3 batch (B=256, its contexts) at 16 q / 2 kv heads,
      head_dim 256: the KV bytes of c3 at twice the head_dim, bf16;
    * ``pi05_bf16`` / ``pi05_fp32``: Pi0.5's attention shape (8 q / 1 kv head,
      head_dim 256), 64 requests with log-uniform [512, 8192] contexts (seed 5),
      bf16 and fp32 pools (the reference allocates fp32 pools for fp32
      models, kv_cache_engine.py:104-105).
    Kernel times per launch from HIP graph replays; algorithmic bytes as for
    the step's decode kernel (KV of every token, q read, o write, indices)."""
    c3 = S.make_batch("c3")
    g = torch.Generator().manual_seed(5)
    u = torch.rand(64, generator=g, dtype=torch.float64).numpy()
    pi_lens = np.rint(np.exp(np.log(512) + u * (np.log(8192) - np.log(512)))).astype(np.int64)
    return {
        "kernel": "decode_kernel<*, false, 256> / attend_f32_kernel<256, false>",
        "how": "HIP graph replay of 4 decode launches of one plan; decode_plus_merge_us adds the merge launches",
        "d256_c3_bytes": _side_decode(dev, steps, 16, 2, 256, c3.kv_len.astype(np.int64), torch.bfloat16, 2),
        "pi05_bf16": _side_decode(dev, steps, 8, 1, 256, pi_lens, torch.bfloat16, 5),
        "pi05_fp32": _side_decode(dev, steps, 8, 1, 256, pi_lens, torch.float32, 5),
    }


def short_rows(bt) -> int:
    """The library's short-query threshold (rows per request) for this batch's shape."""
    s = bt.spec
    return _lib.lib().mi_prefill_short_rows(len(bt.kv_len), s.num_qo_heads, s.num_kv_heads, s.head_dim)


def prefill_flops(bt) -> tuple[int, int]:
    """(flops of the MFMA-tile requests, flops of the short-query requests) of one causal step.

    4*D*Hq flops per visible (query, key) pair: q.k and p.v, a multiply-add each.
    Requests with qo_len*G at most ``mi_prefill_short_rows`` rows run on the decode kernel.
    """
    s = bt.spec
    g = s.num_qo_heads // s.num_kv_heads
    short = short_rows(bt)
    long_f = short_f = 0
    for kvl, qo in zip(bt.kv_len.tolist(), bt.new_len.tolist()):
        pairs = qo * (kvl - qo) + qo * (qo + 1) // 2
        f = 4 * s.head_dim * s.num_qo_heads * pairs
        if qo * g > short:
            long_f += f
        else:
            short_f += f
    return long_f, short_f


def bench_prefill(args, dev) -> dict:
    from mstar_amd.paged_attention import PagedPrefillWrapper

    _log(f"setup {args.config} ...")
    bt = S.make_batch(args.config)
    s = bt.spec
    b = len(bt.kv_len)
    ntok = bt.total_q_tokens
    kv = torch.empty(1, s.pool_pages, 2, s.page_size, s.num_kv_heads, s.head_dim, dtype=torch.bfloat16, device=dev)
    fill_pool(kv, s, dev)
    layer = kv[0]
    g = torch.Generator().manual_seed(s.seed + 1)
    q = torch.randn(ntok, s.num_qo_heads, s.head_dim, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(ntok, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(ntok, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(dev)
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    w = PagedPrefillWrapper(ws, s.num_qo_heads, s.num_kv_heads, s.head_dim, s.page_size, device=dev)
    meta = [torch.from_numpy(a) for a in (bt.qo_indptr, bt.kv_indptr, bt.kv_indices, bt.last_page_len)]

    def step(events=None):
        w.plan(*meta, causal=True)
        w.set_kv_cache(layer, k, v)
        if events is None:
            return w.run(q, layer)
        return _prefill_split(w, q, layer, events)

    torch.cuda.synchronize()
    _log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    evs = _kernel_events(args.steps, 3)
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    tile_ms = np.array([e1.elapsed_time(e2) for _, e1, e2 in evs])
    short_ms = np.array([e0.elapsed_time(e1) for e0, e1, _ in evs])
    long_f, short_f = prefill_flops(bt)
    tile_s = float(tile_ms.mean()) / 1e3
    achieved = long_f / tile_s / 1e12
    short_bytes = 0
    g_ = s.num_qo_heads // s.num_kv_heads
    short = short_rows(bt)
    for kvl, qo in zip(bt.kv_len.tolist(), bt.new_len.tolist()):
        if qo * g_ <= short:
            short_bytes += kvl * s.num_kv_heads * s.head_dim * 2 * 2 + qo * s.num_qo_heads * s.head_dim * 2 * 2
    res = {
        "metric": "ragged prefill+decode attn tokens/s + prefill MFMA TFLOP/s, 1 MI355X",
        "value": ntok / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[s.name],
            "batch": b, "prefill_chunks": s.prefill_chunks, "q_tokens": ntok, "kv_tokens": bt.total_kv_tokens,
            "num_qo_heads": s.num_qo_heads, "num_kv_heads": s.num_kv_heads, "head_dim": s.head_dim,
            "page_size": s.page_size, "causal": True,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
            "traffic": None,
            "kernel": "prefill_kernel",
            "kernel_us": tile_s * 1e6,
            "kernel_us_median": float(np.median(tile_ms)) * 1e3,
            "algorithmic_flops": long_f,
            "short_query_part": {"kernels": "decode_kernel + merge_kernel", "us": float(short_ms.mean()) * 1e3,
                                 "algorithmic_bytes": short_bytes,
                                 "GBps": short_bytes / (float(short_ms.mean()) * 1e-3) / 1e9},
        },
    }
    gemm = library_gemm(dev)
    res["roofline"]["library_gemm"] = gemm
    res["roofline"]["frac_of_library_gemm"] = achieved / gemm["TFLOPs"]
    if not args.no_extra:
        res["prefill_head_dim_256"] = bench_prefill_d256(dev, args.steps)
        res["prefill_fp8_kv"] = bench_prefill_fp8(w, q, layer, s, dev, args.steps, long_f)
        res["prefill_vs_torch_sdpa"] = bench_prefill_vs_sdpa(dev, min(args.steps, 10))
    return res


def bench_prefill_vs_sdpa(dev, steps: int) -> dict:
    """A dense causal GQA prefill (8 sequences of 4096 tokens, 28 q / 4 kv heads,
    head_dim 128, bf16) through PyTorch-ROCm's fused attention
    (``scaled_dot_product_attention(..., enable_gqa=True)``) and through this
    build's paged prefill (8 requests of 4096 new tokens on random pages): the
    same algorithmic flops, HIP events around each call."""
    import torch.nn.functional as F
    from mstar_amd.paged_attention import PagedPrefillWrapper

    b, n, hq, hkv, d, ps = 8, 4096, 28, 4, 128, 16
    flops = 4 * b * hq * d * (n * (n + 1) // 2)
    g = torch.Generator(device=dev).manual_seed(9)
    q = torch.randn(b, hq, n, d, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(b, hkv, n, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(b, hkv, n, d, device=dev, generator=g).to(torch.bfloat16)
    pages = n // ps
    pool = b * pages + 8
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(9)).numpy().astype(np.int32)
    kv_indptr = (np.arange(b + 1) * pages).astype(np.int32)
    last = np.full(b, ps, np.int32)
    qo = (np.arange(b + 1) * n).astype(np.int32)
    cache = torch.empty(pool, 2, ps, hkv, d, device=dev, dtype=torch.bfloat16)
    w = PagedPrefillWrapper(torch.empty(512 << 20, dtype=torch.uint8, device=dev), hq, hkv, d, ps, device=dev)
    w.plan(*(torch.from_numpy(a) for a in (qo, kv_indptr, perm[: b * pages], last)), causal=True)
    qp = q.transpose(1, 2).reshape(b * n, hq, d).contiguous()
    w.set_kv_cache(cache, k.transpose(1, 2).reshape(b * n, hkv, d).contiguous(),
                   v.transpose(1, 2).reshape(b * n, hkv, d).contiguous())
    sdpa = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    ours = lambda: w.run(qp, cache)
    for _ in range(2):
        sdpa()
        ours()
    us_sdpa, us_ours = _run_us(sdpa, steps), _run_us(ours, steps)
    diff = (ours().float() - sdpa().transpose(1, 2).reshape(b * n, hq, d).float()).abs().max().item()
    return {"shape": f"{b} x {n} tokens, {hq} q / {hkv} kv heads, head_dim {d}, causal, bf16",
            "algorithmic_flops": flops,
            "torch_sdpa_us": us_sdpa, "torch_sdpa_frac": flops / us_sdpa / 1e6 / MFMA_BF16_PEAK_TFLOPS,
            "paged_prefill_us": us_ours, "paged_prefill_frac": flops / us_ours / 1e6 / MFMA_BF16_PEAK_TFLOPS,
            "max_abs_diff": diff}


def library_gemm(dev, n: int = 16384, steps: int = 5) -> dict:
    """The box's practical matrix-core ceiling for reference: a square bf16
    GEMM through torch.matmul (hipBLASLt), n^3, HIP events, right after the
    prefill timing (same clock and thermal state)."""
    g = torch.Generator(device=dev).manual_seed(11)
    a = torch.randn(n, n, device=dev, generator=g).to(torch.bfloat16)
    b = torch.randn(n, n, device=dev, generator=g).to(torch.bfloat16)
    for _ in range(2):
        a @ b
    us = _run_us(lambda: a @ b, steps)
    del a, b
    tf = 2 * n ** 3 / us / 1e6
    return {"what": f"torch.matmul bf16 {n}x{n}x{n} (hipBLASLt)", "us": us, "TFLOPs": tf,
            "frac": tf / MFMA_BF16_PEAK_TFLOPS}


def _run_us(fn, steps: int) -> float:
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e3


def bench_prefill_fp8(w, q, layer, s, dev, steps: int, long_flops: int) -> dict:
    """The same planned c4 batch over an fp8-e4m3 copy of the pool (per-head
    scales, the fill_pool quantisation): ``run`` timed whole (short-query
    decode part + prefill tiles) for the bf16 and the fp8 pool."""
    kv8 = torch.empty((1,) + tuple(layer.shape), dtype=torch.float8_e4m3fn, device=dev)
    scales = fill_pool(kv8, s, dev)
    ks, vs = scales[0, 0].contiguous(), scales[0, 1].contiguous()
    l8 = kv8[0]
    for _ in range(2):
        w.run(q, l8, k_scale=ks, v_scale=vs)
    bf = _run_us(lambda: w.run(q, layer), steps)
    f8 = _run_us(lambda: w.run(q, l8, k_scale=ks, v_scale=vs), steps)
    return {"what": "run() of the planned c4 batch, bf16 pool vs fp8-e4m3 pool (in-register dequantisation)",
            "run_us_bf16": bf, "run_us_fp8": f8, "prefill_part_flops": long_flops}


def bench_prefill_d256(dev, steps: int) -> dict:
    """The prefill kernel at head_dim 256 (its own register layout): 8 requests of
    2048 new tokens over 4096..7680-token contexts, 16 q / 2 kv heads, page 16,
    bf16, causal; HIP events around ``run`` (short-query part empty)."""
    from mstar_amd.paged_attention import PagedPrefillWrapper

    hq, hkv, d, ps = 16, 2, 256, 16
    kv_lens = [4096 + 512 * i for i in range(8)]
    new = [2048] * 8
    pages = [-(-n // ps) for n in kv_lens]
    pool = sum(pages) + 8
    perm = np.random.default_rng(0).permutation(pool)
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    kv_indices = perm[: kv_indptr[-1]].astype(np.int32)
    last = np.array([n - (p - 1) * ps for n, p in zip(kv_lens, pages)], np.int32)
    qo = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    g = torch.Generator(device=dev).manual_seed(5)
    cache = torch.randn(pool, 2, ps, hkv, d, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(int(qo[-1]), hq, d, device=dev, generator=g).to(torch.bfloat16)
    w = PagedPrefillWrapper(torch.empty(512 << 20, dtype=torch.uint8, device=dev), hq, hkv, d, ps, device=dev)
    w.plan(*(torch.from_numpy(a) for a in (qo, kv_indptr, kv_indices, last)), causal=True)
    for _ in range(2):
        w.run(q, cache)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        w.run(q, cache)
        b.record()
    torch.cuda.synchronize()
    us = float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e3
    flops = sum(4 * hq * d * (kl - n + t + 1) for kl, n in zip(kv_lens, new) for t in range(n))
    return {"kernel": "prefill_rs_kernel<BF16, false, 256>", "us": us, "algorithmic_flops": flops,
            "TFLOPs": flops / us / 1e6, "frac": flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS}


def _prefill_split(w, q, layer, events):
    """wrapper.run() as its two C entry points, with HIP events around each."""
    desc = _lib.paged_kv_desc(layer)
    out = torch.empty_like(q)
    args = (q.data_ptr(), _lib.MI_BF16, q.stride(0), q.stride(1), desc, w._qo.data_ptr(), w._indptr.data_ptr(),
            w._indices.data_ptr(), w._last.data_ptr(), w._plan_batch, w._plan_max_tokens, w.num_qo_heads, 1,
            1.0 / math.sqrt(w.head_dim), w._workspace.data_ptr(), w._workspace.numel(), out.data_ptr(),
            out.stride(0), out.stride(1), _lib.stream_ptr(q.device))
    e0, e1, e2 = events
    e0.record()
    _lib.check(_lib.lib().mi_prefill_short(*args), "mi_prefill_short")
    e1.record()
    _lib.check(_lib.lib().mi_prefill_tiles(*args), "mi_prefill_tiles")
    e2.record()
    return out


def side_configs(args, dev) -> dict:
    """The other BASELINE configs at full size, compact, for the default run:
    c5 (fp8 KV decode) and c2 (Orpheus decode) as decode-kernel GB/s and
    fraction of HBM peak, c4 (BAGEL ragged prefill + decode) as prefill-kernel
    MFMA fraction plus its short-query decode part.  Each is the same
    measurement as ``--config cN`` (same steps and warm-up, no side
    measurements), run after the headline config's buffers are freed."""
    out = {}
    for name in ("c5", "c2", "c4"):
        sub = argparse.Namespace(**vars(args))
        sub.config = name
        sub.no_extra, sub.no_cpu_baseline = True, True
        torch.cuda.empty_cache()
        if S.SPECS[name].prefill_chunks:
            r = bench_prefill(sub, dev)
            rf = r["roofline"]
            sq = rf["short_query_part"]
            out[name] = {
                "workload": r["config"]["workload"], "steps": sub.steps, "ms_per_step": r["ms_per_step"],
                "tokens_per_s": r["value"],
                "prefill_kernel": rf["kernel"], "prefill_kernel_us": rf["kernel_us"],
                "algorithmic_flops": rf["algorithmic_flops"], "TFLOPs": rf["achieved"],
                "mfma_frac": rf["frac"], "short_query_us": sq["us"], "short_query_bytes": sq["algorithmic_bytes"],
                "short_query_GBps": sq["GBps"], "short_query_hbm_frac": sq["GBps"] / HBM_PEAK_GBS,
                "library_gemm_TFLOPs": rf["library_gemm"]["TFLOPs"],
                "mfma_frac_of_library_gemm": rf["frac_of_library_gemm"],
            }
        else:
            r = bench_decode(sub, dev)
            rf = r["roofline"]
            out[name] = {
                "workload": r["config"]["workload"], "batch": r["config"]["batch"], "kv_dtype": r["config"]["kv_dtype"],
                "steps": sub.steps, "ms_per_step": r["ms_per_step"], "tokens_per_s": r["value"],
                "kernel": rf["kernel"], "kernel_us": rf["kernel_us"], "decode_plus_merge_us": rf["decode_plus_merge_us"],
                "algorithmic_bytes": rf["algorithmic_bytes"], "GBps": rf["achieved"], "hbm_frac": rf["frac"],
                "read_ceiling_GBps": rf["hbm_read_ceiling"]["GBps"], "frac_of_read_ceiling": rf["frac_of_read_ceiling"],
                "same_bytes_read_us": rf["hbm_read_same_bytes"]["us_median"],
                "frac_of_same_bytes_read": rf["frac_of_same_bytes_read"],
            }
        _log(f"{name}: " + json.dumps({k: v for k, v in out[name].items() if k != "workload"}))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the step loop: skip the side measurements (RoPE, KV transfer, "
                         "head_dim 256 and fp8-pool prefill), e.g. for counter runs")
    ap.add_argument("--no-side-configs", action="store_true",
                    help="c3: skip the compact c5 / c2 / c4 measurements that follow the headline")
    ap.add_argument("--trace-ranges", action="store_true",
                    help="decode configs: the manager pushes its tracing ranges (enable_nvtx), for rocprofv3 --marker-trace")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 1 GiB (3x): the reference point that scales "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        return copy_calibration(dev)
    _lib.lib()
    if S.SPECS[args.config].prefill_chunks:
        res = bench_prefill(args, dev)
    else:
        res = bench_decode(args, dev)
    if args.config == "c3" and not args.no_extra and not args.no_side_configs:
        res["configs"] = side_configs(args, dev)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
