"""Benchmark of the semantic block-sparse attention path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 3] [--decode-steps N]

Workload (the headline): one Qwen3.5-4B-shaped full-attention
layer, a 131072-token prompt, 16 query heads / 4 KV heads / head_dim 256, bf16,
synthetic Gaussian-mixture keys and queries (1024 centres, segment lengths
log-uniform in [16, 2048], 4 sink tokens with 8x key norm), K = L/16 = 8192,
query chunk 8192, paper selection settings (tau 0.1, beta 0.25).

A step is one layer's prefill with the inputs resident in HBM: the semantic
block build (spherical k-means per KV head), the packed K/V, and all 16 query
chunks (5 dense-prefix chunks, 11 selected sparse chunks).  ``value`` is that
time in ms per layer.  After the timed steps, the decode step is captured in a
HIP graph N times in a row (256 steps, each with its own query and K/V) and the
graph is replayed: ``decode_us_per_step``.

``roofline`` is for the dominant kernel, the MFMA attention of the prefill:
algorithmic FLOPs (4 D per selected key per query head, plus the causal window
and the dense chunks, counted in one extra pass) over its summed launch time from
HIP events around every launch of the timed steps, on the stream it runs on.  ``decode_roofline`` is the decode step's algorithmic bytes over the
per-step graph time; the bytes of each step come from the clusters that step
selected (an untimed eager run of the same steps writes each step's selected runs).
``cpu_baseline`` times the torch CPU path (the oracle's build and selection, fp32
attention) on the host: a bounded sample of the same layer, a per-step decode
time, and config 1 in full at query chunks 8192 and 1024; it names the CPU model.

After the headline configuration, configurations 2 and 4 (``--extra-configs``)
are measured the same way with ``--extra-steps`` timed prefills and reported
under ``extra_keys`` (no CPU baseline for them).
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "semantic-block-sparse-attention_amd"))
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=None)
    ap.add_argument("--decode-replays", type=int, default=5)
    ap.add_argument("--decode-splits", type=int, default=None,
                    help="splits per KV head of the decode step (default: the runtime config's)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-queries", type=int, default=64)
    ap.add_argument("--only", choices=["all", "prefill", "decode", "dense-alone"], default="all",
                    help="dense-alone: the configuration's dense-prefix chunks by themselves, with no "
                         "index build beside them (for the attention kernel's own counters)")
    ap.add_argument("--extra-configs", type=lambda t: [int(x) for x in t.split(",") if x],
                    default=[2, 4], help="further BASELINE configurations measured after the "
                    "headline one and reported under extra_keys (comma list; empty for none)")
    ap.add_argument("--extra-steps", type=int, default=3,
                    help="timed prefill steps of each extra configuration")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one plain 1 GiB device copy (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return ap.parse_args()


def _log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def run_prefill(layer, inp, conf, timing=None, store_timing=None):
    length = inp.q.shape[0]
    out = torch.empty(length, layer.num_heads * layer.head_dim, dtype=inp.q.dtype,
                      device=inp.q.device)
    if conf.get("order") == "token":
        layer.prefill_token_order(inp.q, inp.q, inp.k, inp.k, inp.v, out, conf["chunk"],
                                  timing=timing, store_timing=store_timing,
                                  fit_tokens=conf["fit_tokens"])
    else:
        layer.prefill(inp.q, inp.q, inp.k, inp.k, inp.v, out, timing=timing)
    return out


def decode_graph(layer, inp, steps, cfg):
    """Capture `steps` consecutive decode steps in one HIP graph (each step reads its own
    query, K/V and position from preloaded device buffers).  Also returns the steps as an
    eager function that writes each step's selected runs (CSR) to a buffer, for the
    per-step byte count (run outside the timed replays)."""
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries
    length = inp.q.shape[0]
    hq, hkv, d = layer.num_heads, layer.num_kv_heads, layer.head_dim
    qs, kn, vn = decode_queries(inp, steps, hq, seed=11)
    qs, kn, vn = qs.cuda(), kn.cuda(), vn.cuda()
    pos = torch.arange(length, length + steps, dtype=torch.int32, device="cuda")
    outs = torch.empty(steps, hq * d, dtype=torch.bfloat16, device="cuda")
    kw = dict(temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
              target_tokens=layer.decode_budget(), sm_scale=layer.scaling,
              num_splits=cfg.decode_num_splits, iters=cfg.iters,
              suffix_splits=cfg.decode_suffix_splits)

    def body(csr=None):
        for t in range(steps):
            fused_decode_step(layer, layer.arena, q_post=qs[t:t + 1], q_pre=qs[t:t + 1],
                              positions=pos[t:t + 1], k_post=kn[t:t + 1], v_states=vn[t:t + 1],
                              output=outs[t:t + 1], csr_out=None if csr is None else csr[t], **kw)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()                               # eager warm-up: workspace, every kernel once
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()

    def selected_rows():
        """Selected prompt rows of every step, summed over the KV heads [steps] (an
        eager run of the same steps, each writing its CSR: rtokens [Hkv] follows
        rstart, rlen, rcum [3, Hkv, C] and rcount [Hkv])."""
        c = layer.index.num_buckets
        csr = torch.zeros(steps, 3 * hkv * c + 2 * hkv, dtype=torch.int32, device="cuda")
        body(csr)
        torch.cuda.synchronize()
        return csr[:, 3 * hkv * c + hkv:].to(torch.int64).sum(dim=1).cpu()

    return graph, outs, selected_rows


def decode_bytes(layer, rows_per_step: torch.Tensor):
    """Algorithmic HBM bytes per captured step, the mean over the steps: per step and KV
    head, the selected rows' K and V (2 D bf16) and their position (each step's own
    count), the suffix rows visible at that step, the descriptors, and the query and
    output rows."""
    idx = layer.index
    hq, hkv, d = layer.num_heads, layer.num_kv_heads, layer.head_dim
    c = idx.num_buckets
    steps = rows_per_step.numel()
    prompt = rows_per_step.double() * (2 * d * 2 + 4)
    suffix = (torch.arange(steps, dtype=torch.float64) + 1) * hkv * 2 * d * 2
    fixed = hkv * c * d * 2 + hq * d * 2 * 2
    per_step = prompt + suffix + fixed
    return float(per_step.mean()), per_step


def cpu_baseline(inp, layer, cfg, sample_queries):
    """The oracle's torch CPU path, timed on the host on a bounded sample.

    Sample: the block build of one KV head over the whole prompt (scaled by Hkv),
    and `sample_queries` queries of the last sparse chunk (selection + sparse
    attention over their selected clusters and window, fp32), scaled to the
    layer's query count.  The dense-prefix chunks are charged at the same
    per-key rate as the sparse attention (keys per query x queries)."""
    from oracle import reference_cpu as ref
    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    length, hq, d = inp.q.shape
    hkv = inp.k.shape[1]
    g = hq // hkv
    k_cpu = inp.k[:, :1].cpu()
    t0 = time.perf_counter()
    product = ref.routing_normalize_keys(k_cpu)
    idx = ref.build_flat_index(product, codebook_seed=0)
    build_s = (time.perf_counter() - t0) * hkv
    # a sample of the last chunk: selection + attention, fp32
    target = layer.target_tokens
    cs = length - cfg.query_chunk_size
    qs = inp.q[cs:cs + sample_queries].cpu()
    k1 = inp.k[:, :1].cpu().float()
    v1 = inp.v[:, :1].cpu().float()
    t0 = time.perf_counter()
    sizes = ref.causal_sizes_at(idx["posting"], idx["indptr"], idx["sizes"], cs)
    vec = ref.trivial_router_vectors(qs[:, :g], 1)
    prob = ref.mixture_probs(vec, None, idx["codebooks"], cfg.selection_temperature)
    sel = ref.theta_select(prob, sizes[None], beta=cfg.bucket_size_penalty, target_tokens=target,
                           g_union=prob.shape[0])["sel"]
    keys_total = 0
    for i in range(qs.shape[0]):
        p = cs + i
        rows = [idx["posting"][0, int(idx["indptr"][0, c]):int(idx["indptr"][0, c]) + int(sizes[0, c])].long()
                for c in torch.nonzero(sel[i, 0]).flatten().tolist()]
        rows.append(torch.arange(cs, p + 1))
        pos = torch.cat(rows)
        kk, vv = k1[pos, 0], v1[pos, 0]
        s = (qs[i, :g].float() @ kk.T) * (d ** -0.5)
        torch.softmax(s, dim=-1) @ vv
        keys_total += pos.numel()
    sample_s = time.perf_counter() - t0
    per_key = sample_s / max(keys_total, 1)              # seconds per (query, key) for G heads
    # keys per query over the layer: dense chunks p+1, sparse chunks ~ K + window
    n_chunks = length // cfg.query_chunk_size
    cap = cfg.dense_prefix_x * target
    total_keys = 0
    for ci in range(n_chunks):
        c0 = ci * cfg.query_chunk_size
        n = cfg.query_chunk_size
        if c0 <= cap:
            total_keys += n * c0 + n * (n + 1) // 2
        else:
            total_keys += n * (keys_total / qs.shape[0] - (sample_queries + 1) / 2) + n * (n + 1) // 2
    attn_s = per_key * total_keys * hkv
    total_ms = (build_s + attn_s) * 1000.0
    # decode: a few steps of the same layer (selection + attention over the selected
    # clusters and the suffix) on the built head, scaled by Hkv
    from semblo_amd.synthetic import decode_queries
    dq, dk, dv = decode_queries(inp, 4, hq, seed=11)
    cluster_of = _cluster_of(idx, length)
    dtimes = cpu_decode(ref, dq[:, :g].cpu(), dk[:, :1].cpu(), dv[:, :1].cpu(), k1, v1, idx,
                        cluster_of, target=target, temperature=cfg.selection_temperature,
                        beta=cfg.bucket_size_penalty, heads=[0])
    decode_ms = 1000.0 * sum(dtimes) / len(dtimes) * hkv
    conf1 = cpu_config1()
    return {"value": round(total_ms, 1), "unit": "ms/layer", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"oracle torch CPU path, fp32: block build of 1 of {hkv} KV heads over the "
                       f"full {length}-token prompt (x{hkv}) and selection + sparse attention of "
                       f"{sample_queries} queries x {g} heads of the last chunk (1 KV head), "
                       f"extrapolated per attended key to all {length} queries and {hkv} KV heads; "
                       f"decode: 4 steps of 1 KV head (x{hkv})"),
            "build_ms": round(build_s * 1000.0, 1), "attention_ms": round(attn_s * 1000.0, 1),
            "decode_ms_per_step": round(decode_ms, 3),
            "config1": conf1}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), as the baseline's report states it."""
    try:
        for text in Path("/proc/cpuinfo").read_text().splitlines():
            if text.startswith("model name"):
                return text.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cluster_of(idx: dict, length: int) -> torch.Tensor:
    """[Hkv, L] cluster of every prompt position: the run of the posting it sits in."""
    posting, indptr, sizes = idx["posting"], idx["indptr"], idx["sizes"]
    hkv, c = sizes.shape
    out = torch.full((hkv, length), -1, dtype=torch.long)
    for h in range(hkv):
        n = sizes[h].long()
        first = torch.repeat_interleave(indptr[h, :c].long(), n)
        rank = torch.arange(int(n.sum())) - torch.repeat_interleave(torch.cumsum(n, 0) - n, n)
        out[h, posting[h, first + rank].long()] = torch.repeat_interleave(torch.arange(c), n)
    return out


def _attend(q, k, v, mask, scale):
    """fp32 attention of q [n, g, d] over k/v [m, d] where mask [n, m] allows."""
    s = torch.einsum("ngd,md->ngm", q, k) * scale
    s.masked_fill_(~mask[:, None, :], float("-inf"))
    return torch.einsum("ngm,md->ngd", torch.softmax(s, dim=-1), v)


def cpu_prefill(ref, q, k, v, idx, cluster_of, *, chunk, target, dense_x, temperature, beta,
                heads, block=1024):
    """The torch CPU path's causal sparse prefill of one layer, fp32: per query chunk,
    dense-prefix chunks attend every earlier key; later chunks select clusters (router,
    mixture probabilities, theta bisection on the causal sizes at the chunk start)
    and attend the selected clusters' earlier keys plus the chunk's own window.  The
    keys of one (chunk, KV head) are gathered once, as the union of the chunk's
    selected clusters; each query masks its own.  Returns the output [L, Hq, D]."""
    length, hq, d = q.shape
    g = hq // k.shape[1]
    scale = d ** -0.5
    out = torch.zeros(length, hq, d)
    pos_all = torch.arange(length)
    for c0 in range(0, length, chunk):
        n = min(chunk, length - c0)
        dense = c0 <= dense_x * target
        sel = None
        if not dense:
            sizes = ref.causal_sizes_at(idx["posting"], idx["indptr"], idx["sizes"], c0)
            vec = ref.trivial_router_vectors(q[c0:c0 + n], 1)
            prob = ref.mixture_probs(vec, None, idx["codebooks"], temperature)
            sel = ref.theta_select(prob, sizes[None], beta=beta, target_tokens=target,
                                   g_union=n)["sel"]
        for h in heads:
            if dense:
                keys = pos_all[:c0 + n]
            else:
                cl = cluster_of[h, :c0]
                union = sel[:, h].any(dim=0)
                keys = torch.cat([pos_all[:c0][union[cl]], pos_all[c0:c0 + n]])
            kk, vv = k[keys, h].float(), v[keys, h].float()
            for b0 in range(0, n, block):
                b1 = min(n, b0 + block)
                p = pos_all[c0 + b0:c0 + b1]
                mask = keys[None, :] <= p[:, None]
                if not dense:
                    before = keys < c0
                    ok = torch.zeros(b1 - b0, keys.numel(), dtype=torch.bool)
                    ok[:, before] = sel[b0:b1, h][:, cluster_of[h, keys[before]]]
                    mask = (mask & ~before[None, :]) | ok
                qq = q[c0 + b0:c0 + b1, h * g:(h + 1) * g].float()
                out[c0 + b0:c0 + b1, h * g:(h + 1) * g] = _attend(qq, kk, vv, mask, scale)
    return out


def cpu_decode(ref, q_steps, k_new, v_new, k, v, idx, cluster_of, *, target, temperature,
               beta, heads):
    """The torch CPU path's decode steps, fp32: per step the query's selection over
    the full clusters, then attention over the selected clusters' keys and the suffix
    keys up to the step.  Returns the seconds of each step."""
    hq, d = q_steps.shape[1:]
    g = hq // k.shape[1]
    scale = d ** -0.5
    times = []
    for t in range(q_steps.shape[0]):
        t0 = time.perf_counter()
        vec = ref.trivial_router_vectors(q_steps[t:t + 1], 1)
        prob = ref.mixture_probs(vec, None, idx["codebooks"], temperature)
        sel = ref.theta_select(prob, idx["sizes"][None], beta=beta, target_tokens=target)["sel"][0]
        for h in heads:
            keys = torch.nonzero(sel[h][cluster_of[h]]).flatten()
            kk = torch.cat([k[keys, h].float(), k_new[:t + 1, h].float()])
            vv = torch.cat([v[keys, h].float(), v_new[:t + 1, h].float()])
            qq = q_steps[t, h * g:(h + 1) * g].float()[None]
            _attend(qq, kk, vv, torch.ones(1, kk.shape[0], dtype=torch.bool), scale)
        times.append(time.perf_counter() - t0)
    return times


def cpu_config1(chunks=(8192, 1024)):
    """Config 1 in full on the host CPU (the torch CPU path, fp32): block build of both
    KV heads, the causal sparse prefill once per query chunk size, and 16 decode
    steps.  One run of each phase (no repetitions)."""
    from oracle import reference_cpu as ref
    from semblo_amd.synthetic import CONFIGS, decode_queries, mixture_layer
    conf = CONFIGS[1]
    length, hq, hkv, d = conf["length"], conf["hq"], conf["hkv"], conf["d"]
    inp = mixture_layer(length, hq, hkv, d, mixtures=conf["mixtures"], seg=conf["seg"],
                        log_uniform=conf["log_uniform"], sinks=conf["sinks"], seed=0,
                        dtype=torch.float32, device="cpu")
    target = length // 16
    t0 = time.perf_counter()
    idx = ref.build_flat_index(ref.routing_normalize_keys(inp.k), codebook_seed=0)
    build_ms = (time.perf_counter() - t0) * 1000.0
    cluster_of = _cluster_of(idx, length)
    res = {"build_ms": round(build_ms, 1)}
    for chunk in chunks:
        t0 = time.perf_counter()
        cpu_prefill(ref, inp.q, inp.k, inp.v, idx, cluster_of, chunk=chunk, target=target,
                    dense_x=4, temperature=0.1, beta=0.25, heads=range(hkv))
        res[f"prefill_ms_chunk{chunk}"] = round((time.perf_counter() - t0) * 1000.0, 1)
    qs, kn, vn = decode_queries(inp, conf["decode_steps"], hq, seed=11, dtype=torch.float32)
    times = cpu_decode(ref, qs.cpu(), kn.cpu(), vn.cpu(), inp.k, inp.v, idx, cluster_of,
                       target=target, temperature=0.1, beta=0.25, heads=range(hkv))
    res["decode_ms_per_step"] = round(1000.0 * sum(times) / len(times), 3)
    res["sample"] = (f"config 1 in full: L={length}, {hq}/{hkv}/{d}, fp32, K={target}; prefill at "
                     f"query chunks {', '.join(map(str, chunks))} (dense-prefix rule x4), "
                     f"{conf['decode_steps']} decode steps; one run of each phase")
    return res


def measured_traffic(config: int):
    """HBM bytes per attention launch (mean over one prefill's launches) from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this configuration, or None."""
    path = ROOT / "profiles" / f"attn_items_kernel_config{config}_traffic.md"
    if not path.exists():
        return None
    for text in path.read_text().splitlines():
        if text.startswith("traffic_bytes_per_launch:"):
            return float(text.split(":", 1)[1])
    return None


def measured_decode_traffic(config: int):
    """HBM bytes per decode step (the step kernel and the merge together) from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this configuration, or None."""
    path = ROOT / "profiles" / f"decode_step_kernel_config{config}_traffic.md"
    if not path.exists():
        return None
    for text in path.read_text().splitlines():
        if text.startswith("traffic_bytes_per_step:"):
            return float(text.split(":", 1)[1])
    return None


def measure(args, config: int, steps: int, warmup: int, with_cpu: bool) -> dict:
    """One configuration: `warmup` + `steps` timed prefills, the captured decode steps,
    and (with_cpu) the CPU baseline.  Returns the bench fields of that configuration."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.kv_outer import KernelTiming
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import CONFIGS, mixture_layer
    conf = CONFIGS[config]
    length, hq, hkv, d = conf["length"], conf["hq"], conf["hkv"], conf["d"]
    dsteps = args.decode_steps if (args.decode_steps is not None and config == args.config) \
        else conf["decode_steps"]
    _log(f"config {config}: L={length} Hq={hq} Hkv={hkv} D={d}")
    inp = mixture_layer(length, hq, hkv, d, mixtures=conf["mixtures"], seg=conf["seg"],
                        log_uniform=conf["log_uniform"], sinks=conf["sinks"], seed=0,
                        dtype=torch.bfloat16, device="cuda")
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                              query_chunk_size=conf["chunk"],
                              suffix_shuffle_seed=5 if conf.get("shuffle_suffix") else None)
    if args.decode_splits:
        cfg.decode_num_splits = max(1, args.decode_splits - cfg.decode_suffix_splits)
    layer = SembloAttention(cfg, layer_name=f"bench.layer.{config}")
    result = {}
    if args.only in ("all", "prefill"):
        # The prefill's host thread waits on the GPU inside the index build, so a
        # full Python garbage collection there (about 20 ms over this process's
        # objects) stalls the layer.  As a serving process does, the objects alive
        # now are collected once and frozen out of later collections; collection
        # itself stays on.  This is done before the warm-up: the step right after a
        # collection runs about 2.5 ms slower, and the warm-up takes that step.
        gc.collect()
        gc.freeze()
        for i in range(warmup):
            run_prefill(layer, inp, conf)
            torch.cuda.synchronize()
            _log(f"warm-up {i} done")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # events between the steps only log the spread, and events around every
        # attention launch time the kernel over the timed steps; nothing waits on them
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        timed = KernelTiming(counts_flops=False)
        marks[0].record()
        for i in range(steps):
            run_prefill(layer, inp, conf, timing=timed)
            marks[i + 1].record()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0 / max(steps, 1)
        gc.unfreeze()
        per_step = [marks[i].elapsed_time(marks[i + 1]) for i in range(steps)]
        _log(f"prefill {ms:.2f} ms/layer (steps on the GPU clock: {', '.join(f'{x:.1f}' for x in per_step)})")
        # one more pass counts the FLOPs of every launch (the same inputs give the
        # same FLOPs in every step) and times the store kernels of a token-order prefill
        timing = KernelTiming()
        store = KernelTiming() if conf.get("order") == "token" else None
        run_prefill(layer, inp, conf, timing=timing, store_timing=store)
        torch.cuda.synchronize()
        attn_ms = timed.total_ms() / max(steps, 1)
        flops = timing.total_flops()
        achieved = flops / (attn_ms * 1e-3) / 1e12
        by_form = {}
        for kind in ("dense", "sparse"):
            ms_k, n_k = timed.split(kind, steps)
            fl_k = timing.split_flops(kind)
            if n_k and ms_k > 0:
                ach = fl_k / (ms_k * 1e-3) / 1e12
                by_form[kind] = {"launches": n_k, "ms": round(ms_k, 3), "tflop": round(fl_k / 1e12, 3),
                                 "achieved": round(ach, 1), "frac": round(ach / PEAK_BF16_TFLOPS, 4)}
        result.update(prefill_ms=ms, attn_ms=attn_ms, flops=flops, achieved=achieved,
                      launches=timing.launches(), by_form=by_form)
        assert timed.launches() == timing.launches() * max(steps, 1)
        _log(f"attention kernel {attn_ms:.2f} ms over {timing.launches()} launches, "
             f"{flops / 1e12:.2f} TFLOP -> {achieved:.1f} TFLOP/s ("
             + ", ".join(f"{k} chunks {v['ms']:.2f} ms, {v['achieved']:.0f} TFLOP/s" for k, v in by_form.items())
             + ")")
        sess = getattr(layer, "last_session", None) if conf.get("order") == "token" else None
        reruns = sess.guard.reruns if sess is not None else getattr(layer, "partials_reruns", 0)
        result.update(partials_reruns=reruns)
        _log(f"sparse chunks run again after passing the partial-buffer cap: {reruns} per layer")
        if store is not None:
            st_ms = store.total_ms()
            st_bytes = store.total_flops()           # the store timing collects bytes
            sess = layer.last_session
            result.update(store_ms=st_ms, store_bytes=st_bytes, store_slices=store.launches() // 2,
                          repacks=sess.repacks, fit_at=sess.fit_at)
            _log(f"store kernels {st_ms:.2f} ms over {store.launches() // 2} appended slices, "
                 f"{st_bytes / 1e9:.2f} GB -> {st_bytes / (st_ms * 1e-3) / 1e9:.0f} GB/s; "
                 f"{sess.repacks} repacks")
    if args.only in ("all", "decode"):
        if layer.arena is None:
            run_prefill(layer, inp, conf)
        graph, outs, selected_rows = decode_graph(layer, inp, dsteps, cfg)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.decode_replays):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / (args.decode_replays * dsteps)
        rows = selected_rows()
        nbytes, per_step_bytes = decode_bytes(layer, rows)
        gbs = nbytes / (us * 1e-6) / 1e9
        result.update(decode_us=us, decode_bytes=nbytes, decode_gbs=gbs,
                      decode_rows_mean=float(rows.double().mean()),
                      decode_rows_min=int(rows.min()), decode_rows_max=int(rows.max()),
                      decode_bytes_min=float(per_step_bytes.min()),
                      decode_bytes_max=float(per_step_bytes.max()))
        _log(f"decode {us:.2f} us/step, {nbytes / 1e6:.1f} MB/step (per step "
             f"{per_step_bytes.min() / 1e6:.1f}-{per_step_bytes.max() / 1e6:.1f}) -> {gbs:.0f} GB/s")
    cpu = None
    if with_cpu and not args.no_cpu_baseline and args.only in ("all", "prefill"):
        cpu = cpu_baseline(inp, layer, cfg, args.cpu_sample_queries)
        _log(f"cpu baseline {cpu['value']} ms/layer on {cpu['cores']} threads")
    if conf.get("order") == "token":
        workload = (f"config {config}: one full-attention layer, L={length}, Hq={hq}, Hkv={hkv}, "
                    f"D={d}, K={layer.target_tokens}, token-order streamed prefill in {conf['chunk']}-"
                    f"token slices, clusters fitted on the first {conf['fit_tokens']} (+1 slice) "
                    f"positions, later keys appended to the fixed clusters; {dsteps} "
                    f"hipGraph-captured decode steps")
    else:
        workload = (f"config {config}: one full-attention layer, L={length}, Hq={hq}, "
                    f"Hkv={hkv}, D={d}, K={layer.target_tokens}, chunk {conf['chunk']}, block build + "
                    f"{length // conf['chunk']}-chunk sparse prefill; {dsteps} hipGraph-captured "
                    f"decode steps")
    fields = {
        "value": round(result.get("prefill_ms", float("nan")), 3),
        "steps": steps,
        "warmup": warmup,
        "config": {"workload": workload, "prompt_tokens": length, "decode_steps": dsteps},
        "decode_us_per_step": round(result["decode_us"], 3) if "decode_us" in result else None,
        "roofline": None if "achieved" not in result else {
            "bound": "mfma", "achieved": round(result["achieved"], 1), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(result["achieved"] / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(config),
            "kernel": "attn_items_kernel<256,4,*> (dense chunks: compact form, sparse chunks: pipelined form)",
            "flops_per_layer": result["flops"], "kernel_ms_per_layer": round(result["attn_ms"], 3),
            "launches_per_layer": result["launches"],
            "partials_reruns": result.get("partials_reruns", 0),
            "by_form": result.get("by_form")},
        "decode_roofline": None if "decode_us" not in result else {
            "bound": "hbm", "achieved": round(result["decode_gbs"], 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(result["decode_gbs"] / PEAK_HBM_GBS, 4),
            "traffic": measured_decode_traffic(config),
            "bytes_per_step": round(result["decode_bytes"]),
            "bytes_per_step_min": round(result["decode_bytes_min"]),
            "bytes_per_step_max": round(result["decode_bytes_max"]),
            "selected_rows_per_step": round(result["decode_rows_mean"], 1),
            "scope": "whole step (select + attend + merge) from graph replay time; bytes from "
                     "each step's own selected runs"},
        "cpu_baseline": cpu,
    }
    if "store_ms" in result:
        gbs = result["store_bytes"] / (result["store_ms"] * 1e-3) / 1e9
        fields["store_roofline"] = {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
            "kernels": "nearest_cluster_kernel + append_rows_kernel + copy_rows_kernel + "
                       "append_index_kernel",
            "kernel_ms_per_layer": round(result["store_ms"], 3),
            "appended_slices": result["store_slices"], "bytes_per_layer": result["store_bytes"],
            "repacks": result["repacks"], "fit_at": result["fit_at"]}
    return fields


def dense_alone(args) -> dict:
    """The dense-prefix chunks of a configuration on their own stream with nothing beside
    them: exact causal attention of each chunk over every earlier position."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.kv_outer import KernelTiming, dense_causal_attention
    from semblo_amd.synthetic import CONFIGS, mixture_layer
    conf = CONFIGS[args.config]
    hq, hkv, d, chunk = conf["hq"], conf["hkv"], conf["d"], conf["chunk"]
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=chunk)
    cap = cfg.dense_prefix_x * cfg.budget(conf["length"])
    length = min(conf["length"], (cap // chunk + 1) * chunk)
    inp = mixture_layer(length, hq, hkv, d, mixtures=conf["mixtures"], seg=conf["seg"],
                        log_uniform=conf["log_uniform"], sinks=conf["sinks"], seed=0,
                        dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(inp.q)
    timing = KernelTiming(counts_flops=False)
    flops = 0.0
    for rep in range(args.warmup + args.steps):
        t = timing if rep >= args.warmup else None
        for cs in range(0, length, chunk):
            n = min(chunk, length - cs)
            if rep == 0:
                flops += 4.0 * d * hq * (n * (cs + 1) + n * (n - 1) // 2)
            dense_causal_attention(inp.q[cs:cs + n], inp.k, inp.v, sm_scale=d ** -0.5, chunk_start=cs,
                                   out=out[cs:cs + n], timing=t)
    torch.cuda.synchronize()
    ms = timing.total_ms() / max(args.steps, 1)
    ach = flops / (ms * 1e-3) / 1e12
    _log(f"dense-prefix chunks alone: {length // chunk} chunks, {ms:.2f} ms, {flops / 1e12:.2f} TFLOP "
         f"-> {ach:.0f} TFLOP/s")
    return {"metric": "dense-prefix chunks alone, ms per layer", "value": round(ms, 3), "unit": "ms",
            "achieved_tflops": round(ach, 1), "frac": round(ach / PEAK_BF16_TFLOPS, 4),
            "config": {"workload": f"config {args.config}: positions 0..{length - 1}, chunk {chunk}"}}


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import semblo_amd
    semblo_amd.load_library()
    if args.only == "dense-alone":
        print(json.dumps(dense_alone(args)), flush=True)
        return
    head = measure(args, args.config, args.steps, args.warmup, with_cpu=True)
    if args.copy_calibration:
        src = torch.empty(1 << 29, dtype=torch.int16, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        _log("copy calibration: 1 GiB read, 1 GiB written")
        del src, dst
    line = {
        "metric": "sparse prefill ms/layer @128K + decode us/step/layer; % MFMA / HBM roofline",
        "value": head["value"],
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["value"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (Gaussian-mixture keys/queries, N(0,1) values, seeded)",
    }
    line.update({k: v for k, v in head.items() if k not in ("value", "steps", "warmup")})
    extra = {}
    for c in args.extra_configs:
        if c == args.config:
            continue
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        f = measure(args, c, args.extra_steps, 1, with_cpu=False)
        extra[f"config{c}"] = {k: v for k, v in f.items() if k != "cpu_baseline"}
    if extra:
        line["extra_keys"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
