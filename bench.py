"""Benchmark of the patched VGGT global-attention layer on one MI355X.

Workload (one step): all 24 global-attention layers of VGGT-1B (dim 1024, 16 heads, d 64, RoPE-2D,
QK-LayerNorm) over 128 frames x 1374 tokens = 175,872 tokens, random-init bf16 weights (seed 0),
N(0,1) input tokens (seed 0); every layer gets its own seeded head table (7 block-top-4 /
4 frame-local / 3 anchor+local / 2 dense, seed 1 + layer), block 64, top-k 4 per frame. Each layer
runs the plugin's HeadwiseSparseAttentionWrapper: qkv Linear -> LayerNorm + RoPE packing -> block
pooling + selection -> single-launch sparse attention -> proj Linear. All inputs are resident in
HBM before timing.

Prints one JSON line: value = effective TFLOP/s of the layer (algorithmic attention FLOP +
projection FLOP per layer / measured time per layer), plus ms per layer, tokens/s, the live
roofline of the sparse attention kernel (algorithmic FLOP per launch / its average duration from
stream events) and a CPU baseline (the oracle's masked fp32 path on the 4-frame shape).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


class EventRecorder:
    """Brackets each kernel launch with events recorded on the current (launching) stream."""

    def __init__(self):
        self.enabled = False
        self.pending = {}
        self.pairs = {}

    def __call__(self, name, phase):
        if not self.enabled:
            return
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        if phase == "start":
            self.pending[name] = ev
        else:
            self.pairs.setdefault(name, []).append((self.pending.pop(name), ev))

    def durations_ms(self):
        torch.cuda.synchronize()
        return {k: [a.elapsed_time(b) for a, b in v] for k, v in self.pairs.items()}


def layer_config(layers, heads, seed_base, synth, ops, table_fn=None):
    """Head-profile config with one seeded block-pattern table per layer (seed ``seed_base + layer``)."""
    names = {ops.BLOCK_DYNAMIC: "block_topk", ops.FRAME_LOCAL: "frame_local", ops.ANCHOR_LOCAL: "anchor_local",
             ops.DENSE: "dense"}
    table_fn = table_fn or synth.seeded_patterns
    cfg, tables = {}, []
    for li in range(layers):
        table = table_fn(heads, seed=seed_base + li)
        tables.append(table)
        groups = {}
        for h, p in enumerate(table):
            groups.setdefault(names[p], []).append(h)
        cfg[str(li)] = [{"mode": m, "head_ids": ids} for m, ids in groups.items()]
    return cfg, tables


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def host_threads() -> int:
    """Cores this process may run on (its affinity set; os.cpu_count() where that is unavailable)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(pkg, frames=4, heads=16, repeats=5, budget_s=25.0):
    """The oracle's fp32 attention path on the 4-frame VGGT shape, timed on the host cores: the masked
    variant (per head, query chunks, full q.k^T plus the pattern's mask) and the gathered variant (keys
    restricted per pattern), both including the block selection; 1 warm-up, then the median of up to
    ``repeats`` runs within ``budget_s`` seconds."""
    import importlib

    from oracle import attention as OA
    from oracle import selection as OS
    synth = importlib.import_module(pkg.__name__ + ".synth")
    acc = importlib.import_module(pkg.__name__ + ".accounting")
    ops = importlib.import_module(pkg.__name__ + ".ops")
    threads = host_threads()
    torch.set_num_threads(threads)
    wl = synth.structured_qkv(frames=frames, heads=heads, seed=0)
    q, k, v = (t.to(torch.bfloat16).float() for t in (wl.q, wl.k, wl.v))
    patterns = synth.round_robin_patterns(heads)
    g = wl.geom
    og = OA.Geometry(g.frames, g.tokens_per_frame, g.num_special)

    def run(gathered):
        sel = {}
        for h, p in enumerate(patterns):
            if p == ops.BLOCK_DYNAMIC:
                sel[h] = torch.from_numpy(OS.block_select(OS.bf16_bits(q[h].numpy()), OS.bf16_bits(k[h].numpy()),
                                                          g.frames, g.tokens_per_frame, g.num_special, 4))
        if gathered:
            outs = [OA.sparse_attention_gathered(q[h], k[h], v[h], p, og, sel.get(h), dtype=torch.float32)
                    for h, p in enumerate(patterns)]
        else:
            outs = [OA.pattern_attention(q[h], k[h], v[h], p, og, sel.get(h), dtype=torch.float32)
                    for h, p in enumerate(patterns)]
        return sel, outs

    def timed(gathered):
        t0 = time.perf_counter()
        sel, _ = run(gathered)  # warm-up
        first = time.perf_counter() - t0
        n = max(1, min(repeats, int(budget_s / 2 / max(first, 1e-3))))
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            run(gathered)
            times.append(time.perf_counter() - t0)
        return sel, statistics.median(times), n

    sel, med, n = timed(False)
    _, med_g, n_g = timed(True)
    dyn = [h for h, p in enumerate(patterns) if p == ops.BLOCK_DYNAMIC]
    sel_t = torch.stack([sel[h] for h in dyn]) if dyn else None
    flops = acc.attention_flops(patterns, g, sel_t)
    return {
        "value": round(flops / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{frames} frames x {g.tokens_per_frame} tokens ({g.tokens}), {heads} heads round-robin "
                   "dense/frame-local/anchor+local/block-top4, oracle masked fp32 attention incl. block selection, "
                   f"no projections; median of {n} runs, {med * 1e3:.0f} ms/layer"),
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "ms_per_layer": round(med * 1e3, 2),
        "gathered_ms_per_layer": round(med_g * 1e3, 2),
        "gathered_value": round(flops / med_g / 1e12, 6),
        "gathered_runs": n_g,
        "algorithmic_flop": flops,
    }


def scores_path(ops, geom, n_dyn, buffers=3):
    """The scores-input selection path (saf3r_topk_from_scores): per-frame top-4 of synthetic fp32
    block-score matrices [n_dyn * NB, NB] (N(0,1) scores), the shape the fused selection scores
    internally. The launches rotate over ``buffers`` distinct matrices (3 x 222 MB at 128 frames, more
    than the 256 MB last-level cache), so each launch reads data the previous launches did not touch;
    every launch is timed by its own stream events."""
    nb = geom.num_blocks
    mats = [torch.randn(n_dyn * nb, nb, device="cuda:0") for _ in range(buffers)]
    idx = ops.topk_from_scores(mats[0], geom.frames, 4)
    torch.cuda.synchronize()
    n = 4 * buffers
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    # the host needs about as long to submit a launch as the GPU to run it: queue every launch behind
    # a GPU spin so that they run back to back, with an event between consecutive launches
    torch.cuda._sleep(50_000_000)
    for r in range(n):
        ev[r].record()
        idx = ops.topk_from_scores(mats[(r + 1) % buffers], geom.frames, 4)
    ev[n].record()
    torch.cuda.synchronize()
    times = [ev[r].elapsed_time(ev[r + 1]) for r in range(n)]
    ms = statistics.median(times)
    nbytes = mats[0].numel() * 4 + idx.numel() * 4
    del mats
    return {"scores_path_ms": round(ms, 4), "scores_path_GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "scores_path_frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "scores_path_note": f"{buffers} rotating {mats_mb(nb, n_dyn)} MB score matrices, cold per launch"}


def mats_mb(nb, n_dyn):
    return round(n_dyn * nb * nb * 4 / 1e6)


def non_lazy_selection(pkg, frames, reps=2):
    """The non-lazy DINO-feature selection at full size: L2-normalised random features
    [frames * 1369, 1024] (the DINOv2-L patch-token width), per-frame top-k through the host mirror of
    compute_qk_topk_indices_batched (bf16 score blocks of 4096 queries, then saf3r_frame_topk_scores),
    for top-4 (the lazy default's k) and top-64 (the paper's non-lazy setting). Also times the
    selection kernel alone on one score block (its HBM rate)."""
    import importlib
    U = importlib.import_module(pkg.__name__ + ".patch.utils")
    ops = importlib.import_module(pkg.__name__ + ".ops")
    P, D = 1369, 1024
    n = frames * P
    g = torch.Generator(device="cuda:0").manual_seed(0)
    feat = torch.nn.functional.normalize(torch.randn(1, n, D, device="cuda:0", generator=g), dim=-1)
    res = {"features": f"{n} x {D}", "gemm_tflop": round(2.0 * n * n * D / 1e12, 2)}
    for k in (4, 64):
        U.compute_qk_topk_indices_batched(feat, feat, k, per_frame=True, num_toks_per_img=P, max_topk=1 << 30)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            U.compute_qk_topk_indices_batched(feat, feat, k, per_frame=True, num_toks_per_img=P, max_topk=1 << 30)
        torch.cuda.synchronize()
        res[f"top{k}_ms"] = round((time.perf_counter() - t0) * 1e3 / reps, 2)
    scores = torch.matmul(feat[0, :4096].to(torch.bfloat16), feat[0].to(torch.bfloat16).t().contiguous())
    ops.frame_topk_scores(scores, frames, P, 64)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        idx = ops.frame_topk_scores(scores, frames, P, 64)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 5
    nbytes = scores.numel() * 2 + idx.numel() * 4
    res["select_block_ms"] = round(ms, 4)
    res["select_block_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    return res


def aggregator_leg(pkg, frames=64, warmup=1, repeats=3, profile=None):
    """The full VGGT-1B-style aggregator forward (DINOv2-L/14 patch embedding, 24 frame + 24 global
    blocks, dim 1024, random-init bf16 weights) over ``frames`` synthetic 518 x 518 frames (uniform [0, 1]
    pixels blurred with a seeded Gaussian, sigma 4): ``warmup`` + ``repeats`` forwards, median ms, first
    with dense global attention (torch SDPA), then with the global attention patched by the plugin with
    the reference's VGGT head profile (lazy dino top-4). The global-attention share is the time between
    stream events recorded around every global ``attn`` module call, over the forward's time."""
    import importlib
    agg = importlib.import_module(pkg.__name__ + ".aggregator")
    plug = importlib.import_module(pkg.__name__ + ".patch")
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    with torch.device(dev):
        model = agg.VGGTAggregatorModel()
    model = model.to(torch.bfloat16).eval()
    images = agg.blurred_frames(frames, 518, 4.0, seed=0, device=dev).to(torch.bfloat16)
    res = {"frames": frames, "image": "518x518", "tokens": frames * 1374,
           "protocol": f"{warmup} warm-up + {repeats} timed forwards, median"}
    # frame blocks and the patch embedding's blocks: torch's fused SDPA where this build has it
    try:
        with torch.no_grad():
            model.aggregator.frame_blocks[0].attn(torch.zeros(2, 1374, 1024, device=dev, dtype=torch.bfloat16),
                                                  pos=model.aggregator.positions(2, 37, 37, dev))
        res["frame_attention"] = "torch SDPA (flash / memory-efficient)"
    except RuntimeError as e:
        model.aggregator.set_frame_attention("saf3r")
        res["frame_attention"] = f"saf3r frame-local kernels (torch SDPA: {str(e)[:80]})"

    def run(tag, patched):
        spans = []

        def pre(mod, args):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            spans.append([ev, None])

        def post(mod, args, out):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            spans[-1][1] = ev

        hooks = []
        for b in model.aggregator.global_blocks:
            hooks.append(b.attn.register_forward_pre_hook(pre))
            hooks.append(b.attn.register_forward_hook(post))
        walls, shares, glob = [], [], []
        try:
            for it in range(warmup + repeats):
                spans.clear()
                torch.cuda.synchronize()
                torch.cuda.reset_peak_memory_stats()
                t0 = time.perf_counter()
                if patched:
                    plug.update_args_per_forward(model, "vggt", 518, 518)
                with torch.no_grad():
                    out, _ = model(images)
                torch.cuda.synchronize()
                dt = (time.perf_counter() - t0) * 1e3
                g_ms = sum(a.elapsed_time(b) for a, b in spans)
                del out
                if it >= warmup:
                    walls.append(dt)
                    glob.append(g_ms)
                    shares.append(g_ms / dt)
        finally:
            for h in hooks:
                h.remove()
        res[tag] = {"forward_ms": round(statistics.median(walls), 1),
                    "global_attn_ms": round(statistics.median(glob), 1),
                    "global_attn_share": round(statistics.median(shares), 4),
                    "peak_mem_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 2)}

    try:
        run("dense", False)
    except RuntimeError as e:
        res["dense"] = f"unavailable: {str(e)[:120]}"
    with open(profile or os.path.join(ROOT, "tests", "golden", "vggt_eth3d_profile.json")) as f:
        prof = json.load(f)
    plug.patch_model(model, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token",
                                                      "lazy_dino_topk": True, "topk": 4}, "sparse_config": prof})
    run("saf3r_lazy_top4", True)
    if isinstance(res.get("dense"), dict):
        res["speedup_vs_dense"] = round(res["dense"]["forward_ms"] / res["saf3r_lazy_top4"]["forward_ms"], 3)
    del model, images
    torch.cuda.empty_cache()
    return res


def calibrate_copy():
    """A plain elementwise copy (negation) of 2^28 fp32 values: 1 GiB read and 1 GiB written once."""
    dev = torch.device("cuda:0")
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kernel": "torch.neg fp32", "read_bytes": src.numel() * 4,
                      "write_bytes": dst.numel() * 4, "launches": 3}), flush=True)


def per_pattern(pkg, frames, reps=5):
    """The attention launch alone, per pattern: 16 heads of one pattern (dense in token order, block
    top-4, frame-local / anchor+local / anchor in the framed layout) and the bench's 16-head mix (seed 1),
    over N(0,1) q / k / v at ``frames`` x 1374 tokens, every head with the softmax scale packed into Q,
    walks paced; 2 warm-up launches, the median of ``reps`` (stream events around each launch)."""
    import importlib
    ops = importlib.import_module(pkg.__name__ + ".ops")
    acc = importlib.import_module(pkg.__name__ + ".accounting")
    synth = importlib.import_module(pkg.__name__ + ".synth")
    dev = torch.device("cuda:0")
    H = 16
    geom = pkg.Geometry(frames, 1374, 5)
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(H, geom.tokens, 64, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    sets = {"dense": [ops.DENSE] * H, "block_topk": [ops.BLOCK_DYNAMIC] * H, "frame_local": [ops.FRAME_LOCAL] * H,
            "anchor_local": [ops.ANCHOR_LOCAL] * H, "anchor": [ops.ANCHOR] * H, "mix": synth.seeded_patterns(H, seed=1)}
    res = {"shape": f"{frames} x 1374 tokens, {H} heads", "reps": reps}
    out = torch.empty(geom.tokens, H * 64, dtype=torch.bfloat16, device=dev)
    for name, pats in sets.items():
        lay = ops.token_order_heads(pats, geom)
        qs = [True] * H
        dyn = [h for h, p in enumerate(pats) if p == ops.BLOCK_DYNAMIC]
        packed = ops.pack_heads(q, k, v, geom, token_order=lay, q_scaled=qs, pool_heads=dyn)
        qp, kp, vp = packed[:3]
        sel = ops.block_select_pooled(packed[-1], frames, geom.blocks_per_frame, 4) if dyn else None
        for _ in range(2):
            ops.sparse_attn_fwd(qp, kp, vp, geom, pats, sel, out=out, token_order=lay, q_scaled=qs)
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            ops.sparse_attn_fwd(qp, kp, vp, geom, pats, sel, out=out, token_order=lay, q_scaled=qs)
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = statistics.median(ts)
        res[name] = {"ms": round(ms, 3), "tflops": round(acc.attention_flops(pats, geom, sel) / (ms * 1e-3) / 1e12, 1)}
        del qp, kp, vp
    return res


def measured_traffic(kernel="sparse_attn_kernel"):
    """HBM bytes per launch of the attention kernel at this workload, as recorded from the
    FETCH_SIZE and WRITE_SIZE counter runs (scaled by the copy calibration) in the committed
    traffic summary; None when that summary is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_vggt1b_global_f128.md")
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(rf"^{kernel}_bytes_per_launch:\s*(\d+)", text, flags=re.M)
    return int(m.group(1)) if m else None


def run_stack(pkg, frames, dim, heads, grid, layers, topk, table_fn, steps, warmup, sparse_cfg=None):
    """The patched global-attention layers of a VGGT-style model on one GPU: ``layers`` layers of
    GlobalAttentionStack(dim, heads) with random-init bf16 weights (seed 0), N(0,1) input tokens (seed 0)
    of ``frames`` frames x (5 + grid^2) tokens, head tables ``table_fn(heads, seed=1 + layer)`` (or the
    head-profile ``sparse_cfg``), block top-``topk``. One step = every layer on the same input, after
    ``update_args_per_forward`` (a new forward). ``warmup`` untimed steps, then ``steps`` timed steps
    between two device synchronisations; stream events bracket every kernel launch of the timed steps."""
    import importlib
    ops = importlib.import_module(pkg.__name__ + ".ops")
    synth = importlib.import_module(pkg.__name__ + ".synth")
    vggt = importlib.import_module(pkg.__name__ + ".vggt")
    plug = importlib.import_module(pkg.__name__ + ".patch")
    acc = importlib.import_module(pkg.__name__ + ".accounting")
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = vggt.GlobalAttentionStack(depth=layers, dim=dim, num_heads=heads)
    model = model.to(dev).to(torch.bfloat16).eval()
    if sparse_cfg is not None:
        plug.patch_model(model, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token",
                                                          "lazy_dino_topk": True, "topk": 4},
                                         "sparse_config": sparse_cfg})
    else:
        cfg, _ = layer_config(layers, heads, 1, synth, ops, table_fn)
        plug.patch_model(model, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token",
                                                          "block_topk": topk, "topk_scope": "frame"},
                                         "sparse_config": cfg})
    plug.update_args_per_forward(model, "vggt", grid * 14, grid * 14)
    T = grid * grid + 5
    N = frames * T
    geom = pkg.Geometry(frames, T, 5)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(1, N, dim, generator=g, device=dev).to(torch.bfloat16)
    pos = synth.vggt_positions(frames, grid, grid, device=dev)[None]
    wrappers = [b.attn for b in model.aggregator.global_blocks]

    def step():
        plug.update_args_per_forward(model, "vggt", grid * 14, grid * 14)  # a new forward: lazy indices recomputed
        for layer in wrappers:
            layer(x, pos)

    rec = EventRecorder()
    ops.set_event_recorder(rec)
    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        rec.enabled = True
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        rec.enabled = False
    ops.set_event_recorder(None)
    ms_step = (t1 - t0) * 1e3 / steps

    # algorithmic work of every layer (selection lists and key sets of the last step); the attention
    # kernel's own share excludes the image rows of dino_topk heads (done by the gather kernel)
    def layer_work(w, full):
        width = w.est_topk_idx.shape[1] if (full and w.dino_heads) else 0
        counts = w.last_keysets.count.tolist() if w.keyset_heads else None
        return acc.attention_flops(w.patterns, geom, w.last_selection, width, counts)

    res = {
        "ms_step": ms_step, "ms_layer": ms_step / layers, "dur": rec.durations_ms(), "layers": wrappers,
        "geom": geom, "model": model, "x": x, "pos": pos,
        "attn_flops": [layer_work(w, True) for w in wrappers],
        "kernel_flops": [layer_work(w, False) for w in wrappers],
        "exec_flops": [acc.executed_tile_flops(w.patterns, geom, w.last_selection,
                                               w.last_keysets.count.tolist() if w.keyset_heads else None,
                                               ops.token_order_heads(w.patterns)) for w in wrappers],
    }
    return res


def pool_increment(run, reps=30, burst=4):
    """What pooling adds to the pack: the first layer's pack (LayerNorm, RoPE, layouts, scaled Q) with
    and without the block records of its block_topk heads, alternated ``reps`` times; each time
    ``burst`` packs run back to back between two stream events (the GPU stays busy, so the host's
    launch work between the packs is not timed). Medians of the per-pack times and of the
    differences of adjacent bursts (which drift of the clock between bursts affects least), in ms."""
    w, x, pos, geom = run["layers"][0], run["x"], run["pos"], run["geom"]
    ts = {True: [], False: []}
    with torch.no_grad():
        qkv = w.orig_module.qkv(x).reshape(geom.tokens, -1).contiguous()
        for pool in (True, False):
            w.pack(qkv, pos, geom, pool)
        torch.cuda.synchronize()
        for _ in range(reps):
            for pool in (True, False):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(burst):
                    w.pack(qkv, pos, geom, pool)
                e1.record()
                torch.cuda.synchronize()
                ts[pool].append(e0.elapsed_time(e1) / burst)
    del qkv
    diffs = [a - b for a, b in zip(ts[True], ts[False])]
    return statistics.median(ts[True]), statistics.median(ts[False]), statistics.median(diffs)


def da3_leg(pkg, steps, warmup):
    """The DA3-Giant-style shape through the plugin: 24 layers, dim 1536, 24 heads, 96 frames of
    5 + 36 x 36 tokens (124,896), per-layer head tables of 12 block-top-8 / 4 frame-local / 4 anchor+local /
    4 dense heads (seed 1 + layer), random-init bf16 weights, N(0,1) tokens."""
    import importlib
    synth = importlib.import_module(pkg.__name__ + ".synth")
    acc = importlib.import_module(pkg.__name__ + ".accounting")
    layers, dim = 24, 1536
    run = run_stack(pkg, 96, dim, 24, 36, layers, 8, synth.da3_patterns, steps, warmup)
    geom = run["geom"]
    attn_ms = run["dur"].get("sparse_attn", [])
    proj = acc.projection_flops(geom.tokens, dim)
    layer_flops = sum(run["attn_flops"]) / layers + proj
    attn_tflops = sum(run["kernel_flops"]) * steps / (sum(attn_ms) * 1e-3) / 1e12
    res = {
        "workload": (f"DA3-Giant-style global attention: {layers} layers x 96 frames x {geom.tokens_per_frame} "
                     f"tokens ({geom.tokens}), 24 heads, d 64, dim 1536, head mix 12 block-top8 / 4 frame-local / "
                     "4 anchor+local / 4 dense per layer (seed 1+layer), block 64"),
        "steps": steps, "warmup": warmup,
        "ms_per_layer": round(run["ms_layer"], 3),
        "tokens_per_s": round(geom.tokens / (run["ms_layer"] * 1e-3), 1),
        "layer_tflops": round(layer_flops / (run["ms_layer"] * 1e-3) / 1e12, 2),
        "attn_ms_per_layer": round(statistics.fmean(attn_ms), 3),
        "attn_tflops": round(attn_tflops, 2),
        "roofline_frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
        "flop_per_layer": {"attention": round(sum(run["attn_flops"]) / layers), "projection": proj},
        "other_kernels_ms": {k: round(statistics.fmean(v), 4) for k, v in run["dur"].items() if k != "sparse_attn"},
    }
    del run
    torch.cuda.empty_cache()
    return res


def single_layer_leg(pkg, frames, reps=10):
    """One global-attention layer on the structured Q/K/V generator (seed 0) at ``frames`` x 1374 tokens,
    16 heads, head table of seed 1 (7 block-top-4 / 4 frame-local / 3 anchor+local / 2 dense): packing
    (Q with the softmax scale, the plugin's layouts, block means), block selection and the attention
    launch, as the wrapper runs them; 2 warm-up layers, the median of ``reps`` (stream events)."""
    import importlib
    ops = importlib.import_module(pkg.__name__ + ".ops")
    synth = importlib.import_module(pkg.__name__ + ".synth")
    acc = importlib.import_module(pkg.__name__ + ".accounting")
    dev = torch.device("cuda:0")
    H = 16
    wl = synth.structured_qkv(frames=frames, heads=H, seed=0, device=dev)
    geom = wl.geom
    q, k, v = (t.to(torch.bfloat16) for t in (wl.q, wl.k, wl.v))
    del wl
    pats = synth.seeded_patterns(H, seed=1)
    lay = ops.token_order_heads(pats, geom)
    qs = [True] * H
    dyn = [h for h, p in enumerate(pats) if p == ops.BLOCK_DYNAMIC]
    out = torch.empty(geom.tokens, H * 64, dtype=torch.bfloat16, device=dev)

    def layer():
        qp, kp, vp, pooled = ops.pack_heads(q, k, v, geom, token_order=lay, q_scaled=qs, pool_heads=dyn)
        sel = ops.block_select_pooled(pooled, frames, geom.blocks_per_frame, 4)
        ops.sparse_attn_fwd(qp, kp, vp, geom, pats, sel, out=out, token_order=lay, q_scaled=qs)
        return sel

    rec = EventRecorder()
    ops.set_event_recorder(rec)
    for _ in range(2):
        layer()
    torch.cuda.synchronize()
    layer_ms = []
    rec.enabled = True
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        sel = layer()
        e1.record()
        torch.cuda.synchronize()
        layer_ms.append(e0.elapsed_time(e1))
    rec.enabled = False
    ops.set_event_recorder(None)
    dur = rec.durations_ms()
    flops = acc.attention_flops(pats, geom, sel)
    ms = statistics.median(layer_ms)
    attn = statistics.median(dur["sparse_attn"])
    return {
        "workload": (f"one global-attention layer, {frames} frames x 1374 tokens ({geom.tokens}), 16 heads, d 64, "
                     "structured Q/K/V (seed 0), head mix 7 block-top4 / 4 frame-local / 3 anchor+local / 2 dense "
                     "(seed 1), block 64; packing with block means + selection + attention, no projections"),
        "reps": reps,
        "ms_per_layer": round(ms, 3),
        "tokens_per_s": round(geom.tokens / (ms * 1e-3), 1),
        "layer_tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "attn_ms": round(attn, 3),
        "attn_tflops": round(flops / (attn * 1e-3) / 1e12, 2),
        "roofline_frac": round(flops / (attn * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "algorithmic_flop": flops,
        "other_kernels_ms": {k: round(statistics.median(v), 4) for k, v in dur.items() if k != "sparse_attn"},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--frames", type=int, default=128)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sparse-config", default=None,
                    help="a head-profile JSON in the reference's format (e.g. its VGGT ETH3D profile) to run "
                         "instead of the seeded block-pattern tables; dino_topk heads use lazy top-4 indices")
    ap.add_argument("--non-lazy-select", action="store_true",
                    help="also time the non-lazy DINO-feature token selection at the full frame count")
    ap.add_argument("--aggregator-frames", type=int, default=64,
                    help="frames of the full-aggregator forward leg (0 skips it)")
    ap.add_argument("--per-pattern", action="store_true",
                    help="run only the per-pattern attention timing (16 heads of each pattern, and the head mix)")
    ap.add_argument("--no-extra-configs", dest="extra_configs", action="store_false",
                    help="skip the 32-frame single-layer and the DA3-Giant-shape legs")
    ap.add_argument("--only-config", choices=["32-frames", "da3-giant"], default=None,
                    help="run only one of the extra legs (the 32-frame single layer or the DA3-Giant shape) and "
                         "print its JSON, for profiling that shape alone")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain copy kernel of known size (reads 1 GiB, writes 1 GiB), for scaling "
                         "the FETCH_SIZE / WRITE_SIZE counters of a profiling run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported (the path is measured on one "
              "MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.per_pattern:
        print(json.dumps({"per_pattern": per_pattern(__graft_entry__.package(), args.frames)}), flush=True)
        return
    if args.only_config == "32-frames":
        print(json.dumps({"config_32_frames": single_layer_leg(__graft_entry__.package(), 32)}), flush=True)
        return
    if args.only_config == "da3-giant":
        print(json.dumps({"config_da3_giant": da3_leg(__graft_entry__.package(), args.steps, args.warmup)}), flush=True)
        return

    import importlib
    pkg = __graft_entry__.package()
    ops = importlib.import_module(pkg.__name__ + ".ops")
    synth = importlib.import_module(pkg.__name__ + ".synth")
    acc = importlib.import_module(pkg.__name__ + ".accounting")

    sparse_cfg = None
    if args.sparse_config:
        with open(args.sparse_config) as f:
            sparse_cfg = {k: v for k, v in json.load(f).items() if int(k) < args.layers}
    run = run_stack(pkg, args.frames, 1024, 16, 37, args.layers, 4, synth.seeded_patterns, args.steps, args.warmup,
                    sparse_cfg)
    ms_step, ms_layer, dur, layers, geom = run["ms_step"], run["ms_layer"], run["dur"], run["layers"], run["geom"]
    N, T, dim, heads = geom.tokens, geom.tokens_per_frame, 1024, 16
    tables = [w.patterns for w in layers]
    attn_flops, kernel_flops, exec_flops = run["attn_flops"], run["kernel_flops"], run["exec_flops"]
    proj = acc.projection_flops(N, dim)
    layer_flops = sum(attn_flops) / args.layers + proj
    attn_ms = dur.get("sparse_attn", [])
    attn_ms_avg = statistics.fmean(attn_ms) if attn_ms else float("nan")
    attn_tflops = (sum(kernel_flops) * args.steps) / (sum(attn_ms) * 1e-3) / 1e12 if attn_ms else None
    n_dyn = sum(1 for p in tables[0] if p == ops.BLOCK_DYNAMIC)
    other_ms = {k: round(statistics.fmean(v), 4) for k, v in dur.items() if k not in ("sparse_attn",)}
    if n_dyn:
        sel_extra_scores = scores_path(ops, geom, n_dyn)
    else:
        sel_extra_scores = {}
    width = args.frames * min(4, geom.blocks_per_frame)
    sb = acc.selection_bytes(geom, n_dyn, width)
    sel_ms = dur.get("block_select", [])
    sel_extra = {}
    if sel_ms:
        pooled_ms, plain_ms, inc = pool_increment(run)
        sel_avg = statistics.fmean(sel_ms)
        fused = max(inc, 0.0) + sel_avg
        sel_extra = {
            "select_kernel": "block_select_mfma_kernel",
            "select_ms": round(sel_avg, 4),
            "pack_ms_with_pooling": round(pooled_ms, 4),
            "pack_ms_without_pooling": round(plain_ms, 4),
            "pool_increment_ms": round(inc, 4),
            "fused_path_ms": round(fused, 4),
            "fused_path_GBs": round(sb["fused_path"] / (fused * 1e-3) / 1e9, 1),
            "fused_path_frac": round(sb["fused_path"] / (fused * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "fused_path_bytes": sb["fused_path"],
            "fused_path_note": ("algorithmic bytes (read Q and K of the block_topk heads, write their lists) over the "
                                "selection's added time: the pack's increment for the block means (median difference "
                                "of 30 adjacent pairs of bursts of 4 back-to-back packs with / without them, a "
                                "negative value counted as 0) plus the selection kernel"),
            "heads": n_dyn,
        }
        sel_extra.update(sel_extra_scores)
    result = {
        "metric": "ms per global-attn layer + effective TFLOP/s, VGGT shape 128 frames bf16",
        "value": round(layer_flops / (ms_layer * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "ms_per_layer": round(ms_layer, 3),
        "tokens_per_s": round(N / (ms_layer * 1e-3), 1),
        "attn_ms_per_layer": round(attn_ms_avg, 3),
        "attn_tflops": None if attn_tflops is None else round(attn_tflops, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) tokens and random-init bf16 weights (seed 0), seeded head tables",
        "config": {
            "workload": (f"VGGT-1B global attention: {args.layers} layers x {args.frames} frames x {T} tokens "
                         f"({N}), 16 heads, d 64, dim 1024, RoPE-2D + QK-LayerNorm, "
                         + (f"head profile {os.path.basename(args.sparse_config)} (lazy dino top-4)"
                            if args.sparse_config else
                            "head mix 7 block-top4 / 4 frame-local / 3 anchor+local / 2 dense per layer "
                            "(seed 1+layer), block 64")),
            "frames": args.frames, "tokens": N, "layers": args.layers, "heads": heads, "block": 64, "topk": 4,
            "parallelism": "single GPU",
        },
        "flop_per_layer": {"attention": round(sum(attn_flops) / args.layers), "projection": proj},
        "roofline": {
            "bound": "mfma",
            "kernel": "sparse_attn_kernel",
            "achieved": None if attn_tflops is None else round(attn_tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": None if attn_tflops is None else round(attn_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": ("FETCH_SIZE + WRITE_SIZE counter runs of this workload, scaled by a copy kernel: "
                               "profiles/hbm_traffic_vggt1b_global_f128.md"),
            "launch_ms": round(attn_ms_avg, 3),
            "executed_tile_flop": round(sum(exec_flops) / args.layers),
            "algorithmic_flop": round(sum(kernel_flops) / args.layers),
            "executed_frac": (None if attn_tflops is None else
                              round(sum(exec_flops) * args.steps / (sum(attn_ms) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)),
        },
        "selection": dict(sel_extra, bound="hbm", peak=PEAK_HBM_GBS, unit="GB/s"),
        "other_kernels_ms": other_ms,
    }
    if args.non_lazy_select:
        result["non_lazy_selection"] = non_lazy_selection(pkg, args.frames)
    del layers, run
    torch.cuda.empty_cache()
    if not args.sparse_config and args.extra_configs:
        result["config_32_frames"] = single_layer_leg(pkg, 32)
        result["config_da3_giant"] = da3_leg(pkg, max(1, args.steps // 4), 1)
    if args.aggregator_frames > 0 and not args.sparse_config:
        result["aggregator"] = aggregator_leg(pkg, args.aggregator_frames)
    if not args.no_cpu_baseline and not args.sparse_config:
        result["cpu_baseline"] = cpu_baseline(pkg)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
