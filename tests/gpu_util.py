"""Shared helpers of the GPU parity tests (selection near-tie accounting, fp64 references)."""
from __future__ import annotations

import math

import torch

from oracle import reference_cpu as ref

# Tolerances of the attention outputs (bf16), from the build's contract.
ATOL = 2e-2
RTOL = 1e-2
# A selection difference is a near-tie when the cluster's score lies within this
# relative margin of the cut (theta) of either run.
NEAR_TIE_REL = 1e-4


def bf16_rounding_near_ties(got: torch.Tensor, want: torch.Tensor, exact: list,
                            rel: float = NEAR_TIE_REL, row_scaled: bool = False) -> int:
    """Values where two bf16 results differ must be rounding near-ties: the two values are
    adjacent bf16 numbers and one of the ``exact`` candidates (fp64, the quantity before
    the rounding, one tensor per rounding stage that can flip) lies within ``rel`` of the
    midpoint between them.  The margin is relative to the value itself; with
    ``row_scaled`` (vectors, such as unit keys and centroids, whose elements can cancel to
    nearly zero) it is relative to the larger of the value and the RMS of its row (last
    dimension), and two results that both lie within that margin of the exact value also
    pass.  Returns how many values differ."""
    gf = got.cpu().float()
    wf = want.cpu().float()
    g = gf.double().flatten()
    w = wf.double().flatten()
    diff = torch.nonzero(g != w).flatten()
    if diff.numel() == 0:
        return 0
    gb = got.cpu().contiguous().view(torch.int16).flatten()[diff].int()
    wb = want.cpu().contiguous().view(torch.int16).flatten()[diff].int()
    adjacent = ((gb - wb).abs() == 1) & ((gb ^ wb) >= 0)       # same sign, one ulp apart
    mid = 0.5 * (g[diff] + w[diff])
    ok = torch.zeros_like(adjacent)
    for e in exact:
        ed = e.cpu().double().expand(gf.shape)
        x = ed.flatten()[diff]
        if row_scaled:
            rms = ed.pow(2).mean(-1, keepdim=True).sqrt().expand(gf.shape).flatten()[diff]
            scale = torch.maximum(x.abs(), rms)
            ok |= adjacent & ((x - mid).abs() <= rel * scale)
            ok |= ((g[diff] - x).abs() <= rel * rms) & ((w[diff] - x).abs() <= rel * rms)
        else:
            ok |= adjacent & ((x - mid).abs() <= rel * mid.abs())
    bad = ~ok
    assert not bool(bad.any()), (
        f"{int(bad.sum())} of {diff.numel()} differing bf16 values are not rounding near-ties "
        f"within {rel} (first at flat index {int(diff[bad][0])}: got {float(g[diff][bad][0])!r}, "
        f"want {float(w[diff][bad][0])!r})")
    return int(diff.numel())


def assert_close_bf16(got: torch.Tensor, want: torch.Tensor, what: str = "") -> float:
    g = got.double().cpu()
    w = want.double().cpu()
    err = (g - w).abs()
    bad = err > ATOL + RTOL * w.abs()
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} values off by more than "
        f"{ATOL} + {RTOL}*|ref| (max err {float(err.max()):.4g})")
    return float(err.max())


def compare_selection(sel_gpu: torch.Tensor, sel_ref: torch.Tensor, score: torch.Tensor,
                      theta_ref: torch.Tensor, theta_gpu: torch.Tensor | None = None) -> dict:
    """sel_* [Q, Hkv, C] bool, score [Q, Hkv, C] (oracle scores), theta [Q, Hkv].

    Every differing cluster must be a near-tie: its score within NEAR_TIE_REL
    (relative) of theta, plus the bisection's resolution (range * 2^-16).
    Returns counts for the report.
    """
    sel_gpu = sel_gpu.cpu()
    sel_ref = sel_ref.cpu()
    diff = sel_gpu != sel_ref
    n_diff = int(diff.sum())
    if n_diff == 0:
        return {"differ": 0, "near_ties": 0, "pairs": int(sel_ref.shape[0] * sel_ref.shape[1])}
    live = score > -1e38
    big = torch.full_like(score, 1e38)
    rng = score.max(-1).values - torch.where(live, score, big).min(-1).values
    slack = rng.clamp_min(0) * 2.0 ** -16
    thetas = [theta_ref.cpu()]
    if theta_gpu is not None:
        thetas.append(theta_gpu.cpu())
    ok = torch.zeros_like(diff)
    for th in thetas:
        tol = NEAR_TIE_REL * th.abs().clamp_min(1.0) + slack
        ok |= (score - th[..., None]).abs() <= tol[..., None]
    bad = diff & ~ok
    assert not bool(bad.any()), (
        f"{int(bad.sum())} selection differences are not near-ties, e.g. "
        f"{torch.nonzero(bad)[:5].tolist()}")
    return {"differ": n_diff, "near_ties": n_diff, "pairs": int(sel_ref.shape[0] * sel_ref.shape[1])}


def attention_reference(q: torch.Tensor, keys_pos: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        sm_scale: float) -> torch.Tensor:
    """fp64 softmax attention. q [Q, Hq, D]; keys_pos bool [Q, Hkv, L] (the key set of every
    query and KV head); k/v [L, Hkv, D] in prompt order."""
    qd = q.double()
    kd = k.double()
    vd = v.double()
    qn, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = torch.zeros(qn, hq, d, dtype=torch.float64)
    for h in range(hkv):
        s = torch.einsum("qgd,ld->qgl", qd[:, h * g:(h + 1) * g], kd[:, h]) * sm_scale
        m = keys_pos[:, h][:, None, :]
        s = s.masked_fill(~m, -math.inf)
        p = torch.softmax(s, dim=-1)
        out[:, h * g:(h + 1) * g] = torch.einsum("qgl,ld->qgd", p, vd[:, h])
    return out


def cluster_position_mask(posting: torch.Tensor, indptr: torch.Tensor, counts: torch.Tensor,
                          length: int) -> torch.Tensor:
    """[Hkv, C, L] bool: the positions of the first counts[h, c] rows of cluster c's run."""
    hkv, c = counts.shape
    m = torch.zeros(hkv, c, length, dtype=torch.bool)
    for h in range(hkv):
        for cl in range(c):
            s = int(indptr[h, cl])
            n = int(counts[h, cl])
            if n:
                m[h, cl, posting[h, s:s + n].long()] = True
    return m


def oracle_select(vectors, codebooks, sizes, *, temperature, beta, target, g_union=None, sink=0):
    """The oracle's scores and bisection; one size snapshot ([1, Hkv, C]) serves every query.
    ``sink`` > 0: cluster 0 hidden from the search, the budget less the sink, then cluster
    0 selected for every query (fused_prefill.py:382-405)."""
    prob = ref.mixture_probs(vectors.cpu(), None, codebooks.cpu(), temperature)
    if g_union is None:
        g_union = prob.shape[0] if sizes.shape[0] == 1 else 1
    sizes = sizes.cpu()
    if sink:
        sizes, target = ref.hold_out_sink(sizes, target, sink)
    out = ref.theta_select(prob, sizes, beta=beta, target_tokens=target, g_union=max(g_union, 1))
    if sink:
        out["sel"][..., 0] = True
        ref.force_sink_bit(out["qmask"], out["bitmask"])
    return out


# ---------------------------------------------------------------- k-means trace ----------

def bf16_midpoint_gap(v: torch.Tensor) -> torch.Tensor:
    """|v - m| (fp64) for the bf16 rounding midpoint m between the two bf16 numbers around
    v: the value where round-to-nearest changes its result."""
    bits = v.float().view(torch.int32)
    mid = ((bits & ~0xFFFF) | 0x8000).view(torch.float32).double()
    return (v.double() - mid).abs()


def assignment_near_ties(x_bf16: torch.Tensor, cent_bf16: torch.Tensor, got: torch.Tensor,
                         want: torch.Tensor, rel: float = NEAR_TIE_REL) -> int:
    """Rows whose argmax cluster differs between two implementations that both take the
    first maximum of the bf16-rounded similarity (fp32 sums in different orders).  A flip
    between clusters a and b is a near-tie when their rounded similarities are equal or
    adjacent bf16 numbers and the exact (fp64) similarity of a or b lies within ``rel``
    (relative) of a bf16 rounding midpoint: only there can a reordered fp32 sum round the
    other way.  Asserts every flip is one; returns how many rows flipped."""
    rows = torch.nonzero(got != want).flatten()
    if rows.numel() == 0:
        return 0
    x = x_bf16[rows].double()
    c = cent_bf16.double()
    sg = (x * c[got[rows]]).sum(-1)
    sw = (x * c[want[rows]]).sum(-1)
    rg = sg.float().to(torch.bfloat16).float().double()
    rw = sw.float().to(torch.bfloat16).float().double()
    mag = torch.maximum(rg.abs(), rw.abs()).clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    adjacent = (rg - rw).abs() <= ulp * 1.0001
    near = torch.minimum(bf16_midpoint_gap(sg), bf16_midpoint_gap(sw)) <= rel * mag
    bad = ~(adjacent & near)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} of {rows.numel()} assignment flips are not near-ties, e.g. row "
        f"{int(rows[bad][0])}: sims {float(sg[bad][0]):.8g} / {float(sw[bad][0]):.8g}")
    return int(rows.numel())


def check_fit_trace(product_h: torch.Tensor, gpu: dict, ref_steps: list, ref_final: torch.Tensor,
                    ref_final_centroids: torch.Tensor, tag: str = "",
                    k_pre_h: torch.Tensor | None = None) -> dict:
    """Each k-means step of one KV head's GPU build against the oracle fed the GPU's own
    inputs, then the GPU's trajectory against the oracle's own.

    product_h [L, I] bf16 (the router's keys of the head); ``gpu`` one entry of the build's
    ``fit_trace``; ``ref_steps`` the oracle's per-iteration states for the same head
    (fit_flat_codebook(steps=...)); ``ref_final`` its final assignment [L] and
    ``ref_final_centroids`` its final fp32 centroids; ``k_pre_h`` the pre-RoPE keys when
    the GPU build ran the router itself (router_pass), so that rows whose router output
    differs can be traced to a router rounding near-tie.

    Step parity (every difference a counted near-tie, else the test fails):
      * key space: fp32 within 2e-6 of the oracle's (or the row's router output differs
        at a rounding near-tie), bf16 rounding near-ties;
      * per iteration, given the GPU's centroids: the assignment (argmax flips at
        near-ties), the counts exactly, the sums to fp32 summation order, and the next
        centroids (bf16 rounding near-ties of the exact centroids);
      * the final assignment of every key given the GPU's final centroids.
    Trajectory: while the GPU's states equal the oracle's, any difference in the bf16
    centroids must be a rounding near-tie of the exact centroid (counted as an origin).
    A GPU build that leaves the oracle's trajectory must do so at a counted near-tie
    (key space, centroid rounding or assignment flip); otherwise its final assignment
    may differ from the oracle's only by the final near-ties.
    """
    import torch.nn.functional as F
    space_ref = F.normalize(ref.routing_space(product_h).float(), dim=-1)
    exact_space = F.normalize(product_h.double(), dim=-1)
    far = (gpu["space_f32"] - space_ref).abs().amax(-1) > 2e-6
    n_router = int(far.sum())
    if n_router:
        # rows whose router output (bf16) differs: the GPU build normalised the pre-RoPE
        # keys itself, and some element of the row must be a rounding near-tie there
        assert k_pre_h is not None, f"{tag}: key space differs from the oracle's ({n_router} rows)"
        r = F.normalize(k_pre_h[far].double(), dim=-1)
        rms = r.pow(2).mean(-1, keepdim=True).sqrt()
        near = (bf16_midpoint_gap(r) <= NEAR_TIE_REL * torch.maximum(r.abs(), rms)).any(-1)
        assert bool(near.all()), \
            f"{tag}: {int((~near).sum())} key rows differ with no router rounding near-tie"
    keep = ~far
    n_space = bf16_rounding_near_ties(gpu["space_bf16"][keep], space_ref.to(torch.bfloat16)[keep],
                                      [exact_space[keep]], row_scaled=True)
    sample = gpu["sample"]
    xs_bf = gpu["space_bf16"][sample]
    xs_f32 = gpu["space_f32"][sample]
    xs_ref = space_ref[sample]
    c = gpu["entry_centroids"][0].shape[0]

    def onehot_sums64(x, assign):
        return torch.zeros(c, x.shape[1], dtype=torch.float64).index_add_(0, assign, x.double())

    flips_assign = flips_cent = 0
    origin = int((xs_bf != xs_ref.to(torch.bfloat16)).any(-1).sum())   # sample rows whose bf16 differs
    on_track = origin == 0
    first_departure = -1
    iters = len(gpu["assign"])
    for i in range(iters):
        cin = gpu["entry_centroids"][i]
        a_gpu = gpu["assign"][i]
        if on_track:
            # same states so far: the entry centroids against the oracle's own
            n = bf16_rounding_near_ties(cin, ref_steps[i]["entry"].to(torch.bfloat16),
                                        ([exact_entry] if i else []) + [ref_steps[i]["entry"]],
                                        row_scaled=True)
            origin += n
            on_track = n == 0
        a_ref = ref.argmax_sim_chunked(xs_bf.float(), cin.float(), 65536)
        n = assignment_near_ties(xs_bf, cin, a_gpu, a_ref)
        flips_assign += n
        if on_track:
            origin += n
            on_track = n == 0
        if first_departure < 0 and not torch.equal(a_gpu, ref_steps[i]["assign"]):
            first_departure = i
        counts = torch.bincount(a_gpu, minlength=c)
        assert torch.equal(gpu["counts"][i].long(), counts), f"{tag}: counts at iteration {i}"
        sums = ref.segment_sum_matmul(xs_f32, a_gpu, c)
        scale = counts.clamp_min(1).double()[:, None]
        assert float(((gpu["sums"][i].double() - sums.double()).abs() / scale).max()) <= 1e-5, \
            f"{tag}: sums at iteration {i}"
        live = counts > 0
        nxt = gpu["entry_centroids"][i + 1] if i + 1 < iters else gpu["final_centroids"]
        cent = F.normalize(sums / counts.clamp_min(1)[:, None].float(), dim=-1)
        exact_entry = F.normalize(onehot_sums64(xs_ref, a_gpu) / scale, dim=-1)
        flips_cent += bf16_rounding_near_ties(nxt[live], cent[live].to(torch.bfloat16),
                                              [exact_entry[live],
                                               F.normalize(onehot_sums64(xs_f32, a_gpu) / scale,
                                                           dim=-1)[live]], row_scaled=True)
    if on_track:
        n = bf16_rounding_near_ties(gpu["final_centroids"], ref_final_centroids.to(torch.bfloat16),
                                    [exact_entry], row_scaled=True)
        origin += n
    fin = ref.argmax_sim_chunked(gpu["space_bf16"].float(), gpu["final_centroids"].float(), 65536)
    flips_final = assignment_near_ties(gpu["space_bf16"], gpu["final_centroids"],
                                       gpu["final_assign"], fin)
    moved = int((gpu["final_assign"] != ref_final).sum())
    rep = dict(router_flips=n_router, space_flips=n_space, assign_flips=flips_assign, centroid_flips=flips_cent,
               final_flips=flips_final, origin_flips=origin, first_departure=first_departure,
               moved=moved)
    if origin == 0:
        assert first_departure < 0, f"{tag}: left the oracle's trajectory at no near-tie: {rep}"
        # the same final centroids: keys outside the sample differ only at final near-ties
        # or where their own bf16 key space differs
        space_moved = int((gpu["space_bf16"] != space_ref.to(torch.bfloat16)).any(-1).sum())
        assert moved <= flips_final + space_moved, f"{tag}: {rep}"
    return rep


# ---------------------------------------------------------------- sparse chunks ----------

def sparse_rows_reference(q_rows: torch.Tensor, qpos: torch.Tensor, sel: torch.Tensor,
                          sizes: torch.Tensor, posting: torch.Tensor, indptr: torch.Tensor,
                          k: torch.Tensor, v: torch.Tensor, wstart: int,
                          sm_scale: float) -> torch.Tensor:
    """fp64 attention of some queries of a sparse chunk over exactly their key sets
    (kv_outer.py:482-816): the first sizes[h, c] rows of every selected cluster c plus
    the causal window wstart..p.  q_rows [n, Hq, D] at positions qpos [n]; sel [n, Hkv, C]
    bool; k/v [L, Hkv, D] in prompt order.  Returns [n, Hq, D] fp64."""
    n, hq, d = q_rows.shape
    hkv, c = sizes.shape
    g = hq // hkv
    runs = [[posting[h, int(indptr[h, cl]):int(indptr[h, cl]) + int(sizes[h, cl])].long()
             for cl in range(c)] for h in range(hkv)]
    out = torch.zeros(n, hq, d, dtype=torch.float64)
    for i in range(n):
        p = int(qpos[i])
        win = torch.arange(wstart, p + 1)
        for h in range(hkv):
            cl = torch.nonzero(sel[i, h]).flatten().tolist()
            keys = torch.cat([runs[h][x] for x in cl] + [win])
            s = q_rows[i, h * g:(h + 1) * g].double() @ k[keys, h].double().T * sm_scale
            out[i, h * g:(h + 1) * g] = torch.softmax(s, dim=-1) @ v[keys, h].double()
    return out


def causal_rows_reference(q_rows: torch.Tensor, qpos: torch.Tensor, k: torch.Tensor,
                          v: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """fp64 causal attention of some queries (positions qpos) over keys 0..p."""
    n, hq, d = q_rows.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = torch.zeros(n, hq, d, dtype=torch.float64)
    for i in range(n):
        p = int(qpos[i])
        for h in range(hkv):
            s = q_rows[i, h * g:(h + 1) * g].double() @ k[:p + 1, h].double().T * sm_scale
            out[i, h * g:(h + 1) * g] = torch.softmax(s, dim=-1) @ v[:p + 1, h].double()
    return out


def decode_rows_reference(q: torch.Tensor, packed: torch.Tensor, indptr: torch.Tensor,
                          sizes: torch.Tensor, sel: torch.Tensor, suffix_k: torch.Tensor,
                          suffix_v: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """ref.decode_reference with the packed store left on the device: only the selected
    runs come to the host."""
    hkv = packed.shape[2]
    rows, starts = [], torch.zeros(hkv, indptr.shape[1] - 1, dtype=torch.int64)
    total = 0
    for h in range(hkv):
        for cl in torch.nonzero(sel[h]).flatten().tolist():
            starts[h, cl] = total
            n = int(sizes[h, cl])
            rows.append(torch.arange(int(indptr[h, cl]), int(indptr[h, cl]) + n))
            total += n
    idx = torch.cat(rows) if rows else torch.zeros(0, dtype=torch.int64)
    small = packed[:, idx.to(packed.device)].cpu()
    ip = torch.zeros(hkv, indptr.shape[1], dtype=torch.int64)
    ip[:, :-1] = starts
    return ref.decode_reference(q, small, ip, sizes, sel, suffix_k, suffix_v, sm_scale)


def check_recorded_chunk(rec: dict, q: torch.Tensor, q_pre: torch.Tensor, k: torch.Tensor,
                         v: torch.Tensor, index, out: torch.Tensor, *, target: int,
                         rows: torch.Tensor | None = None, tau: float = 0.1, beta: float = 0.25,
                         tag: str = "", sink: int = 0) -> dict:
    """One sparse chunk of a prefill, from its recorded plan (ChunkPlan.record): the
    attention of the sampled rows against fp64 over the GPU's own key sets, with no
    query off tolerance, and the GPU's selection against the oracle's (differences only
    at counted near-ties).  q, q_pre, k, v, out: CPU tensors of the whole prompt."""
    cs, ce, wstart = rec["chunk_start"], rec["chunk_end"], rec["wstart"]
    sizes = rec["causal_sizes"].cpu()
    hkv, c = sizes.shape
    qmask = rec["qmask"].cpu()
    n = ce + 1 - cs
    if rows is None:
        rows = torch.arange(n)
    sel = ref.unpack_bits(qmask[rows], c)
    want = sparse_rows_reference(q[cs + rows], cs + rows, sel, sizes,
                                 index.posting_positions.cpu(), index.bucket_indptr.cpu(),
                                 k, v, wstart, q.shape[-1] ** -0.5)
    err = assert_close_bf16(out[cs + rows], want, f"{tag} chunk {cs}")
    vec = ref.trivial_router_vectors(q_pre[cs + rows], 1)
    exp = oracle_select(vec, index.codebooks.cpu(), sizes[None], temperature=tau, beta=beta,
                        target=target, sink=sink)
    theta = rec["theta"].cpu()[rows] if rec.get("theta") is not None else None
    rep = compare_selection(sel, exp["sel"], exp["score"], exp["theta"], theta)
    rep["max_err"] = err
    return rep
