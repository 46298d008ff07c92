#!/usr/bin/env python3
"""Benchmark of the mixed INT8/BF16 tile linear path on one MI355X.

Workload ("M=4 decode"): the Llama-3.2-3B decoder
linear set -- Q/K/V (stacked, 5120x3072), O (3072x3072), Gate/Up (stacked,
16384x3072), Down (3072x8192) -- for all 28 layers, 4 tokens, a seeded
uniform keep01 tile mask per projection, W ~ N(0, 0.02) bf16, activations
N(0, 1) with 0.5% outlier channels x20.  A step is one pass of the hot path
(activation quantization + mixed tile GEMM) through the 112 projections of
the 28 layers: 2.85 GB of distinct packed weights, well above the 256 MB
Infinity Cache.  The step is captured once as a HIP graph and replayed.

Prints ONE JSON line: value = whole-job TOPS (2*tokens*M*K summed over the
step / step time); roofline = the GEMM kernel's packed-weight GB/s against
8 TB/s HBM, from HIP events around a graph of the step's GEMM launches run
back to back (per-launch average); cpu_baseline = the
CPU oracle (oracle/tq_oracle.c, the reference's arithmetic) on a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HIDDEN, KV, MLP, LAYERS = 3072, 1024, 8192, 28
HBM_PEAK_GBPS = 8000.0
# projection groups of one decoder layer: (name, member output widths, K)
GROUPS = (("qkv", (HIDDEN, KV, KV), HIDDEN), ("o", (HIDDEN,), HIDDEN),
          ("gate_up", (MLP, MLP), HIDDEN), ("down", (HIDDEN,), MLP))
# the decoder-layer modules of each group's members (Decision/ stems: model.layers.<i>.<member>)
MEMBERS = (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), ("self_attn.o_proj",),
           ("mlp.gate_proj", "mlp.up_proj"), ("mlp.down_proj",))
# released Llama-3.2-3B gi tile maps (Decision/meta-llama_Llama-3.2-3B-Instruct/gi/tile_masks/keepXX,
# committed as test fixtures)
RELEASED_MAPS = ROOT / "tests" / "golden"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=4)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--keep", type=float, default=0.01)
    ap.add_argument("--cpu-layers", type=int, default=4, help="layers in the CPU baseline sample (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="minimum CPU work timed for the baseline")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense bf16 context measurement")
    ap.add_argument("--prefill-tokens", type=int, default=8192, help="prefill measurement rows (0 = skip)")
    ap.add_argument("--prefill-keep", type=float, default=0.05)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--e2e", type=int, default=1, help="end-to-end generation section (BASELINE configs[4]); 0 = skip")
    ap.add_argument("--e2e-only", action="store_true", help="run only the end-to-end section (profiling)")
    ap.add_argument("--prefill-only", action="store_true", help="run only the prefill section (profiling)")
    ap.add_argument("--qwen", type=int, default=1, help="Qwen2.5-7B/14B shapes section (BASELINE configs[3]); 0 = skip")
    ap.add_argument("--qwen-only", action="store_true", help="run only the Qwen section (profiling)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the decode GEMM launches (3 eager steps) and a 256 MiB copy: the workload of "
                         "the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes behind roofline.traffic")
    ap.add_argument("--attention-traffic-probe", action="store_true",
                    help="run only three eager decode-attention calls (RoPE form with the INT8 merge; B=4, 24/8 "
                         "heads, 2304 keys) and a 256 MiB copy: the workload of the FETCH_SIZE pass behind "
                         "profiles/decode_attention_traffic.md")
    ap.add_argument("--decode-glue-probe", action="store_true",
                    help="run only graph timings of the fused decode step's glue kernels (configs[4] decode shape): "
                         "residual add + RMSNorm + codes, SiLU * up + codes, and the RoPE attention split + INT8 "
                         "merge over 28 distinct caches; microseconds per launch")
    ap.add_argument("--trace-split", metavar="KERNEL_TRACE_CSV",
                    help="per-layer split of the prompt forwards in a rocprofv3 kernel trace (no GPU needed)")
    ap.add_argument("--traffic-summarize", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="read the two --pmc passes' counter_collection.csv and write " + TRAFFIC_FILE)
    ap.add_argument("--released-maps", type=int, default=1,
                    help="also measure decode and prefill with the released Llama-3.2-3B gi tile maps; 0 = skip")
    ap.add_argument("--released-only", action="store_true", help="run only the released-maps section")
    ap.add_argument("--m-sweep", type=int, default=1,
                    help="also time the decode linear set at 1, 16 and 64 tokens (BASELINE configs[1]); 0 = skip")
    ap.add_argument("--config0", type=int, default=1,
                    help="BASELINE configs[0]: one 3072->3072 MixedLinear at 16 tokens, GPU beside the CPU path")
    ap.add_argument("--e2e-batch", type=int, default=4)
    ap.add_argument("--e2e-prompt", type=int, default=2048)
    ap.add_argument("--e2e-output", type=int, default=256)
    ap.add_argument("--e2e-warmup", type=int, default=2)
    ap.add_argument("--e2e-repeats", type=int, default=5)
    ap.add_argument("--e2e-dense-eager", type=int, default=1)
    ap.add_argument("--e2e-dense", type=int, default=1, help="also run the dense bf16 baseline model")
    ap.add_argument("--e2e-module-path", type=int, default=1,
                    help="also time both models with the modules' own forward in the decode graph")
    return ap.parse_args()


TRAFFIC_FILE = "profiles/decode_gemm_traffic.json"
TRAFFIC_COPY_BYTES = 256 << 20
GEMM_KERNEL = "tq::gemm_decode_kernel"


def _counter_rows(d):
    import csv
    import glob
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def traffic_summarize(args):
    """HBM bytes per decode GEMM launch from two rocprofv3 --pmc passes of
    --traffic-probe (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each
    scaled by what the same counter reads for the probe's plain copy of
    TRAFFIC_COPY_BYTES (read once, written once)."""
    def per_kernel(rows, counter):
        gemm, copy = [], []
        for r in rows:
            if r["Counter_Name"] != counter:
                continue
            v = float(r["Counter_Value"])
            if GEMM_KERNEL in r["Kernel_Name"]:
                gemm.append(v)
            elif "neg_kernel" in r["Kernel_Name"] and int(r["Grid_Size"]) >= (TRAFFIC_COPY_BYTES >> 6):
                copy.append(v)
        if not gemm or not copy:
            raise SystemExit(f"{counter}: no {GEMM_KERNEL} or copy dispatches found")
        return statistics.mean(gemm), statistics.median(copy), len(gemm)
    fg, fc, n_f = per_kernel(_counter_rows(args.traffic_summarize[0]), "FETCH_SIZE")
    wg, wc, n_w = per_kernel(_counter_rows(args.traffic_summarize[1]), "WRITE_SIZE")
    f_scale = TRAFFIC_COPY_BYTES / (fc * 1024.0)
    w_scale = TRAFFIC_COPY_BYTES / (wc * 1024.0)
    out = {"kernel": GEMM_KERNEL, "tokens": args.tokens, "layers": args.layers, "keep": args.keep,
           "gemm_dispatches": n_f, "fetch_kib_per_dispatch": fg, "write_kib_per_dispatch": wg,
           "copy_bytes": TRAFFIC_COPY_BYTES, "copy_fetch_kib": fc, "copy_write_kib": wc,
           "fetch_scale": f_scale, "write_scale": w_scale,
           "traffic_bytes_per_launch": fg * 1024.0 * f_scale + wg * 1024.0 * w_scale}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


# kernel-name classes of the captured prompt forward (--trace-split) and of the decode step
PREFILL_CLASSES = (("gemm_tilequant", ("gemm_prefill",)), ("gemm_hipblaslt", ("Cijk_",)),
                   ("quantization", ("act_absmax", "act_quant", "act_scales")),
                   ("attention", ("attn_fwd", "flash", "fmha")),
                   ("glue", ("add_rmsnorm_rows", "rope_prefill", "silu_mul_rows")))
DECODE_MARKERS = ("gemm_decode", "attn_split", "attn_merge", "add_rmsnorm_quant", "silu_mul_quant",
                  "argmax_partial", "greedy_finish", "gemm_splitk")


def trace_split(path, layers=LAYERS):
    """Per-layer split of the prompt forwards in a rocprofv3 --kernel-trace
    CSV: prefills are maximal runs of kernels without a decode-step kernel
    that hold a RoPE launch per layer; each one's kernel time by class
    (GEMM, quantization, attention, glue, other) and its GPU span, median
    over the prefills of each model (TileQuant: a prefill with
    gemm_prefill kernels; dense: without)."""
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    segs, cur = [], []
    for start, end, name in rows:
        if any(m in name for m in DECODE_MARKERS):
            if cur:
                segs.append(cur)
            cur = []
        else:
            cur.append((start, end, name))
    if cur:
        segs.append(cur)
    per_model = {"tilequant": [], "dense": []}
    for seg in segs:
        if sum("rope_prefill" in n for _, _, n in seg) < layers:
            continue
        # the prompt forward itself: from its first glue kernel's layer (embedding etc. just before) to the end
        first = next(i for i, (_, _, n) in enumerate(seg) if "add_rmsnorm_rows" in n)
        seg = seg[max(0, first - 2):]
        cls = {c: 0.0 for c, _ in PREFILL_CLASSES}
        cls["other"] = 0.0
        for start, end, name in seg:
            for c, keys in PREFILL_CLASSES:
                if any(k in name for k in keys):
                    cls[c] += (end - start) / 1e6
                    break
            else:
                cls["other"] += (end - start) / 1e6
        model = "tilequant" if cls["gemm_tilequant"] > 0 else "dense"
        span = (seg[-1][1] - seg[0][0]) / 1e6
        per_model[model].append({"span_ms": span, "kernel_ms": cls})
    out = {}
    for model, segs_m in per_model.items():
        if not segs_m:
            continue
        med = lambda xs: statistics.median(xs)   # noqa: E731
        classes = {c: med([s["kernel_ms"][c] for s in segs_m]) for c in segs_m[0]["kernel_ms"]}
        out[model] = {"prefills": len(segs_m), "span_ms": med([s["span_ms"] for s in segs_m]),
                      "kernel_ms": classes, "per_layer_us": {c: v * 1e3 / layers for c, v in classes.items()},
                      "gaps_ms": med([s["span_ms"] - sum(s["kernel_ms"].values()) for s in segs_m])}
    print(json.dumps(out, indent=1))
    return out


def traffic_for(args):
    """roofline.traffic from the committed --pmc summary when it was taken on this workload, else None."""
    try:
        with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if (t.get("kernel"), t.get("tokens"), t.get("layers"), t.get("keep")) != (GEMM_KERNEL, args.tokens,
                                                                           args.layers, args.keep):
        return None
    return t["traffic_bytes_per_launch"]


def keep_ids(n_tr, n_tc, frac, rng):
    import numpy as np

    n = n_tr * n_tc
    k = max(1, int(math.ceil(frac * n)))
    return np.sort(rng.choice(n, size=k, replace=False)).astype(np.int64)


def build_layers(args, device, keep_dir=None, first_layer=0):
    """Pack every projection of every layer with the HIP packer (weights made on
    the GPU).  Tile maps: seeded uniform at args.keep, or the Decision/ archive
    in keep_dir (module names model.layers.<i>.<member>)."""
    import numpy as np
    import torch
    from tilequant_amd.mask_io import load_fp16_keep_ids_for_layer
    from tilequant_amd.mixed_linear import MixedLinear
    from tilequant_amd.pack import concat_packs_along_rows, pack_weight_from_tile_ids

    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")
    rng = np.random.default_rng(args.seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    layers, packed_bytes, ops, t16_total, t8_total, max_row16 = [], 0, 0, 0, 0, 0
    for li in range(first_layer, first_layer + args.layers):
        mods = {}
        for (name, widths, k), members in zip(GROUPS, MEMBERS):
            packs = []
            for m, member in zip(widths, members):
                W = (torch.randn((m, k), generator=gen, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
                n_tr, n_tc = m // 64, k // 64
                if keep_dir is None:
                    ids16 = keep_ids(n_tr, n_tc, args.keep, rng)
                else:
                    ids, grid = load_fp16_keep_ids_for_layer(keep_dir, f"model.layers.{li}.{member}")
                    assert tuple(grid) == (n_tr, n_tc), (member, grid)
                    ids16 = ids.numpy().astype(np.int64)
                mask = np.zeros(n_tr * n_tc, bool)
                mask[ids16] = True
                ids8 = np.flatnonzero(~mask)
                packs.append(pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc,
                                                       int8_tile_ids=torch.from_numpy(ids8),
                                                       fp16_tile_ids=torch.from_numpy(ids16), cfg=cfg))
                del W
            pack = packs[0] if len(packs) == 1 else concat_packs_along_rows(packs)
            lin = MixedLinear(pack, None, cfg)
            t8, t16 = int(pack.int8_tiles.shape[0]), int(pack.fp16_tiles.shape[0])
            t8_total += t8
            t16_total += t16
            packed_bytes += 4096 * t8 + 8192 * t16 + 4 * t8
            ops += 2 * args.tokens * pack.M_orig * pack.K_orig
            rp = pack.fp16_row_ptr.cpu()
            max_row16 = max(max_row16, int((rp[1:] - rp[:-1]).max()))
            mods[name] = lin
        layers.append(mods)
    torch.cuda.synchronize()
    return layers, dict(packed_bytes=packed_bytes, ops=ops, t8=t8_total, t16=t16_total, max_bf16_per_row=max_row16)


def _one_layer_of(args, device, keep_dir, layer_index):
    """build_layers for one decoder layer with the archive's maps of layer layer_index."""
    a2 = argparse.Namespace(**vars(args))
    a2.layers = 1
    return build_layers(a2, device, keep_dir=keep_dir, first_layer=layer_index)


def make_inputs(args, device):
    import torch

    g = torch.Generator(device="cpu")
    g.manual_seed(args.seed + 1)
    xs = {}
    for name, _, k in GROUPS:
        x = torch.randn((args.tokens, k), generator=g)
        ch = torch.randperm(k, generator=g)[: round(0.005 * k)]
        x[:, ch] *= 20
        xs[name] = x.to(torch.bfloat16).to(device)
    return xs


INT8_PEAK_TOPS = 5030.0   # dense INT8 MFMA, 256 CU x 2.4 GHz x 8192 ops/clk

# Qwen2.5 linear shapes (hidden, kv out, mlp)
QWEN = (("qwen2.5-7b", 3584, 512, 18944), ("qwen2.5-14b", 5120, 1024, 13824))
QWEN_MIN_LAYERS = 12


def _groups_of(hidden, kv, mlp):
    return (("qkv", (hidden, kv, kv), hidden), ("o", (hidden,), hidden),
            ("gate_up", (mlp, mlp), hidden), ("down", (hidden,), mlp))


def _clustered_pack(m, k, frac, gen, cpu_gen, device, cfg):
    """A bf16 weight with structure (3% of the 64-column input blocks x4, 3% of
    the 64-row output blocks x3, on top of N(0, 0.02)) and the reference's
    top-k mask on per-tile sum|W| (k = max(1, ceil(frac * tiles)),
    src/quantization/decisions.py:176): the BF16 tiles cluster in those bands,
    so row tiles get very uneven BF16/INT8 mixes."""
    import torch
    from tilequant_amd.pack import pack_weight_from_tile_ids

    n_tr, n_tc = m // 64, k // 64
    W = torch.randn((m, k), generator=gen, device=device, dtype=torch.float32) * 0.02
    cb = torch.randperm(n_tc, generator=cpu_gen)[: max(1, round(0.03 * n_tc))].to(device)
    rb = torch.randperm(n_tr, generator=cpu_gen)[: max(1, round(0.03 * n_tr))].to(device)
    W4 = W.view(n_tr, 64, n_tc, 64)
    W4[:, :, cb, :] *= 4
    W4[rb] *= 3
    W = W.to(torch.bfloat16)
    scores = W.float().abs().view(n_tr, 64, n_tc, 64).sum(dim=(1, 3)).flatten()
    kk = max(1, int(math.ceil(frac * n_tr * n_tc)))
    ids16 = torch.topk(scores, kk).indices.sort().values
    mask = torch.zeros(n_tr * n_tc, dtype=torch.bool, device=device)
    mask[ids16] = True
    ids8 = torch.nonzero(~mask).flatten()
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=ids8.cpu(),
                                     fp16_tile_ids=ids16.cpu(), cfg=cfg)
    del W, scores
    return pack


def qwen_measure(args, device):
    """Qwen2.5-7B / 14B linear shapes with clustered
    keep10 / keep20 masks.  Decode (4 tokens): a HIP graph of quantize + GEMM
    over whole layers, at least QWEN_MIN_LAYERS distinct layers and more than
    512 MB of packed weights; GEMM kernel time from a graph of the GEMM
    launches alone, and per projection group from a graph of that group's
    launches.  Prefill (8192 tokens): one layer through MixedLinear."""
    import statistics as st
    import torch
    from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
    from tilequant_amd.mixed_linear import MixedLinear
    from tilequant_amd.pack import concat_packs_along_rows
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax
    from tilequant_amd.quantize_activation import quantize_activation_token_blocked

    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")
    out = {}
    s = torch.cuda.Stream()

    def graph_time(fn, reps):
        # the side stream must see the inputs the default stream produced (packs, codes)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
        with torch.cuda.stream(s):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / reps   # ms

    for model, hidden, kv, mlp in QWEN:
        groups = _groups_of(hidden, kv, mlp)
        for keep in (0.10, 0.20):
            gen = torch.Generator(device=device)
            gen.manual_seed(args.seed + 11)
            cpu_gen = torch.Generator(device="cpu")
            cpu_gen.manual_seed(args.seed + 12)
            layers, packed, t16, max_row16 = [], 0, 0, 0
            # enough distinct layers that the per-group graphs (one launch per layer) are not
            # dominated by the graph replay's own overhead, and the weights stream cold
            while packed <= 512 * 1024 * 1024 or len(layers) < QWEN_MIN_LAYERS:
                mods = {}
                for name, widths, k in groups:
                    packs = [_clustered_pack(m, k, keep, gen, cpu_gen, device, cfg) for m in widths]
                    pack = packs[0] if len(packs) == 1 else concat_packs_along_rows(packs)
                    mods[name] = MixedLinear(pack, None, cfg)
                    t8, n16 = int(pack.int8_tiles.shape[0]), int(pack.fp16_tiles.shape[0])
                    packed += 4096 * t8 + 8192 * n16 + 4 * t8
                    t16 += n16
                    rp = pack.fp16_row_ptr.cpu()
                    max_row16 = max(max_row16, int((rp[1:] - rp[:-1]).max()))
                layers.append(mods)
            gx = torch.Generator(device="cpu")
            gx.manual_seed(args.seed + 13)
            xs = {name: (torch.randn((4, k), generator=gx) * 1.0).to(torch.bfloat16).to(device) for name, _, k in groups}
            ops = sum(2 * 4 * mods[name].M_orig * mods[name].K_orig for mods in layers for name, _, _ in groups)
            step_ms = graph_time(lambda: [mods[name](xs[name]) for mods in layers for name, _, _ in groups], 10)
            # the codes in the layout MixedLinear gives each projection's GEMM at 4 rows
            blocked = {name: layers[0][name].token_blocked_codes(4) for name, _, _ in groups}
            quant = {name: (quantize_activation_token_blocked if blocked[name] else quantize_activation_tile_absmax)(
                xs[name]) for name, _, _ in groups}
            outs = {(i, name): torch.empty((4, mods[name].M_orig), device=device, dtype=torch.bfloat16)
                    for i, mods in enumerate(layers) for name, _, _ in groups}

            def gemms():
                for i, mods in enumerate(layers):
                    for name, _, _ in groups:
                        lin = mods[name]
                        xq, sx = quant[name]
                        gemm_mixed_rows_splitk(x_fp=xs[name], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                               int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                               int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                               fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr,
                                               M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc,
                                               out_dtype=torch.bfloat16, out=outs[(i, name)],
                                               tile_layout=lin.tile_layout,
                                               x_int8_layout="token_blocked" if blocked[name] else "row_major")
            gemm_ms = graph_time(gemms, 10)
            n_launch = len(layers) * len(groups)
            achieved = packed / n_launch / (gemm_ms / n_launch / 1e3) / 1e9

            # per projection group: its launches of every layer in one graph (cold weights: each
            # layer's copy is distinct), average duration and HBM fraction on its packed bytes
            group_us, group_frac = {}, {}
            for gname, _, _ in groups:
                def group_gemms(gname=gname):
                    for i, mods in enumerate(layers):
                        lin = mods[gname]
                        xq, sx = quant[gname]
                        gemm_mixed_rows_splitk(x_fp=xs[gname], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                               int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                               int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                               fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr,
                                               M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc,
                                               out_dtype=torch.bfloat16, out=outs[(i, gname)],
                                               tile_layout=lin.tile_layout,
                                               x_int8_layout="token_blocked" if blocked[gname] else "row_major")
                us = graph_time(group_gemms, 10) * 1e3 / len(layers)
                lin0 = layers[0][gname]
                gbytes = 4096 * int(lin0.int8_tiles.shape[0]) + 8192 * int(lin0.fp16_tiles.shape[0]) \
                    + 4 * int(lin0.int8_tiles.shape[0])
                group_us[gname] = us
                group_frac[gname] = gbytes / (us / 1e6) / 1e9 / HBM_PEAK_GBPS
            dec = {"layers": len(layers), "packed_bytes": packed, "bf16_tiles": t16,
                   "max_bf16_tiles_per_row_tile": max_row16, "ms_per_step": step_ms,
                   "tops": ops / (step_ms / 1e3) / 1e12, "gbps_packed_weights": packed / (step_ms / 1e3) / 1e9,
                   "gemm_avg_launch_us": gemm_ms * 1e3 / n_launch, "gemm_gbps": achieved,
                   "gemm_hbm_frac": achieved / HBM_PEAK_GBPS, "group_us": group_us, "group_hbm_frac": group_frac}
            del outs, quant
            # prefill: one layer, 8192 tokens
            mods = layers[0]
            pre = {}
            pops = 0
            for name, _, k in groups:
                x = torch.randn((args.prefill_tokens, k), generator=gx).to(torch.bfloat16).to(device)
                lin = mods[name]
                pre[name] = steady_ms(lambda: lin(x))
                pops += 2 * args.prefill_tokens * lin.M_orig * lin.K_orig
                del x
            pms = sum(pre.values())
            out.setdefault(model, {})[f"keep{int(round(keep * 100)):02d}"] = {
                "decode_4tok": dec,
                "prefill": {"tokens": args.prefill_tokens, "layer_ms": pms, "tops": pops / (pms / 1e3) / 1e12,
                            "frac_int8_peak": pops / (pms / 1e3) / 1e12 / INT8_PEAK_TOPS,
                            "group_ms": pre}}
            del layers, mods
            torch.cuda.empty_cache()
    out["data"] = ("random-init weights with 3% of input-column and output-row 64-blocks scaled (x4, x3) and the "
                   "top-k per-tile sum|W| mask; decode activations N(0,1) at 4 tokens")
    return out


PREFILL_REPS = 10
PREFILL_WARM_MS = 50.0


def steady_ms(fn):
    """Median of PREFILL_REPS timed calls of fn (HIP events, synchronised each
    call) after at least PREFILL_WARM_MS of untimed calls: the compute clock
    has ramped up by then, whatever ran before (host-side packing leaves the
    GPU idle, decode work is memory-bound)."""
    import time
    import torch

    t0 = time.perf_counter()
    while True:
        fn()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= PREFILL_WARM_MS:
            break
    times = []
    for _ in range(PREFILL_REPS):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    return statistics.median(times)


def plain_read_launch_us(device, stream, n_launch, nbytes, reps):
    """Per-launch time of a plain HBM read (tq_read_probe) of nbytes, n_launch
    launches over distinct buffers back to back in one HIP graph on stream,
    HIP events around the replays: the GEMM roofline's context (a kernel that
    only reads its bytes, at the same size and in the same protocol)."""
    import torch
    from tilequant_amd import _native as nat

    nbytes = nbytes // 16 * 16
    bufs = torch.empty((n_launch, nbytes), device=device, dtype=torch.uint8)
    sink = torch.zeros((256,), device=device, dtype=torch.int32)

    def reads():
        h = nat.stream_handle(device)
        for i in range(n_launch):
            nat.check(nat.lib().tq_read_probe(nat.ptr(bufs[i]), nbytes, nat.ptr(sink), h), "tq_read_probe")

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        reads()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        reads()
    with torch.cuda.stream(stream):
        for _ in range(2):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * n_launch)
    del g, bufs, sink
    return us


def decode_m_sweep(args, device, layers, info, token_counts=(1, 16, 64)):
    """BASELINE configs[1] at the other token counts it names (M in {1, 4, 16,
    64}; 4 is the headline): the same 28-layer linear set, quantize + GEMM per
    projection in one HIP graph per step, and the GEMM launches alone in a
    graph for the per-launch average (HBM fraction on packed weight bytes)."""
    import torch
    from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax
    from tilequant_amd.quantize_activation import quantize_activation_token_blocked

    s = torch.cuda.Stream()

    def graph_ms(fn, reps):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
        with torch.cuda.stream(s):
            for _ in range(2):
                g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / reps

    out = {}
    n_launch = len(layers) * len(GROUPS)
    for m in token_counts:
        a2 = argparse.Namespace(**vars(args))
        a2.tokens = m
        xs = make_inputs(a2, device)
        step_ms = graph_ms(lambda: [mods[name](xs[name]) for mods in layers for name, _, _ in GROUPS], 10)
        # the codes in the layout MixedLinear gives each projection's GEMM at this row count
        blocked = {name: layers[0][name].token_blocked_codes(m) for name, _, _ in GROUPS}
        quant = {name: (quantize_activation_token_blocked if blocked[name] else quantize_activation_tile_absmax)(
            xs[name]) for name, _, _ in GROUPS}
        outs = [torch.empty((m, mods[name].M_orig), device=device, dtype=torch.bfloat16)
                for mods in layers for name, _, _ in GROUPS]

        def gemms():
            i = 0
            for mods in layers:
                for name, _, _ in GROUPS:
                    lin, (xq, sx) = mods[name], quant[name]
                    gemm_mixed_rows_splitk(x_fp=xs[name], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                           int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                           int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                           fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr,
                                           M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc,
                                           out_dtype=torch.bfloat16, out=outs[i], tile_layout=lin.tile_layout,
                                           x_int8_layout="token_blocked" if blocked[name] else "row_major")
                    i += 1

        gemm_ms = graph_ms(gemms, 10)
        launch_us = gemm_ms * 1e3 / n_launch
        ops = info["ops"] / args.tokens * m   # 2 M K per token over the set
        out[str(m)] = {"ms_per_step": step_ms, "tops": ops / (step_ms / 1e3) / 1e12,
                       "gbps_packed_weights": info["packed_bytes"] / (step_ms / 1e3) / 1e9,
                       "hbm_frac_step": info["packed_bytes"] / (step_ms / 1e3) / 1e9 / HBM_PEAK_GBPS,
                       "gemm_avg_launch_us": launch_us,
                       "gemm_hbm_frac": info["packed_bytes"] / n_launch / (launch_us / 1e6) / 1e9 / HBM_PEAK_GBPS,
                       "token_blocked_codes": sorted(name for name, b in blocked.items() if b)}
        del quant, outs, xs
    return out


def prefill_measure(args, device, keep_dir=None):
    """one Llama-3.2-3B layer's QKV/O/GateUp/Down at
    prefill_tokens rows (MixedLinear: whole-input scales, default row chunk),
    keep05 uniform masks (or, with keep_dir, the released map of the layer
    whose row tiles carry the most BF16 tiles).  Compute-bound: reported
    against INT8 MFMA peak."""
    import numpy as np
    import torch

    a2 = argparse.Namespace(**vars(args))
    a2.layers, a2.keep, a2.tokens = 1, args.prefill_keep, args.prefill_tokens
    if keep_dir is None:
        layers, info = build_layers(a2, device)
    else:
        best = None
        for li in range(args.layers):   # pick the layer with the most BF16 tiles in one row tile
            from tilequant_amd.mask_io import load_fp16_keep_ids_for_layer

            worst = 0
            for members in MEMBERS:
                for member in members:
                    ids, (n_tr, n_tc) = load_fp16_keep_ids_for_layer(keep_dir, f"model.layers.{li}.{member}")
                    worst = max(worst, int(np.bincount(ids.numpy() // n_tc, minlength=n_tr).max()) if ids.numel() else 0)
            if best is None or worst > best[1]:
                best = (li, worst)
        layers, info = _one_layer_of(a2, device, keep_dir, best[0])
    g = torch.Generator(device="cpu")
    g.manual_seed(args.seed + 7)
    xs = {name: torch.randn((args.prefill_tokens, k), generator=g).to(torch.bfloat16).to(device)
          for name, _, k in GROUPS}
    mods = layers[0]
    per = {name: steady_ms(lambda name=name: mods[name](xs[name])) for name, _, _ in GROUPS}
    total_ms = sum(per.values())
    return {"tokens": args.prefill_tokens, "keep": args.prefill_keep if keep_dir is None else f"released {keep_dir.name}",
            "max_bf16_tiles_per_row_tile": info["max_bf16_per_row"], "layer_ms": total_ms,
            "tops": info["ops"] / (total_ms / 1e3) / 1e12,
            "frac_int8_peak": info["ops"] / (total_ms / 1e3) / 1e12 / INT8_PEAK_TOPS,
            "group_ms": per, "ops_per_layer": info["ops"], "bf16_tiles": info["t16"],
            "note": "MixedLinear forward per group (scales over all rows, then one quantize + one "
                    f"GEMM), HIP events, median of {PREFILL_REPS} after {PREFILL_WARM_MS:.0f} ms of warm-up calls"}


LLAMA32_3B = dict(vocab_size=128256, hidden_size=HIDDEN, intermediate_size=MLP, num_hidden_layers=LAYERS,
                  num_attention_heads=24, num_key_value_heads=8, head_dim=128, rope_theta=5e5, rms_norm_eps=1e-5,
                  max_position_embeddings=131072, tie_word_embeddings=True)


def _dense_model(config, device, seed, dtype):
    """Random-init dense bf16 model of the same architecture (the baseline), materialised on the device."""
    import torch
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM

    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(config, dtype=dtype, attn_implementation="sdpa")
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for name, p in list(model.named_parameters()):
        mod_name, _, leaf = name.rpartition(".")
        owner = model.get_submodule(mod_name) if mod_name else model
        if "norm" in mod_name.lower():
            value = torch.ones(p.shape, device=device, dtype=dtype)
        else:
            value = (torch.randn(p.shape, generator=gen, device=device, dtype=torch.float32) * 0.02).to(dtype)
        owner._parameters[leaf] = torch.nn.Parameter(value, requires_grad=False)
    for mod in model.modules():
        for bname, buf in list(mod._buffers.items()):
            if buf is not None and buf.device != device:
                mod._buffers[bname] = buf.to(device)
    model.tie_weights()
    return model.eval()


def _energy_reader():
    """Function returning the GPU's accumulated energy in microjoules (amdsmi,
    the counterpart of the reference's NVML counter), or None when amdsmi is
    unavailable on this host."""
    try:
        import amdsmi

        amdsmi.amdsmi_init()
        handle = amdsmi.amdsmi_get_processor_handles()[0]

        def read():
            try:
                e = amdsmi.amdsmi_get_energy_count(handle)
                return float(e["energy_accumulator"]) * float(e["counter_resolution"])
            except Exception:
                return None

        return read if read() is not None else (lambda: None)
    except Exception:
        return lambda: None


def e2e_measure(args, device):
    """BASELINE configs[4] / the reference's benchmark protocol
    (examples/benchmark_generation.py:74-155): random-init Llama-3.2-3B
    architecture, every decoder linear a MixedLinear with a seeded uniform
    keep01 tile map, greedy generation through the HIP-graph decoder; batch 4,
    2048 seeded uniform prompt ids, 256 output tokens.  TTFT = request start to
    first token (host prompt copy included), TPOT = (end - first) / (O - 1),
    tok/s = B * O / (end - start); medians over the timed requests.  The dense
    bf16 model of the same architecture runs the reference's eager loop and the
    same graph decoder."""
    import gc

    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from transformers import LlamaConfig
    from tilequant_amd.api import build_mixed_precision_model
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder
    from tilequant_amd.types import ApplyConfig

    B, P, O = args.e2e_batch, args.e2e_prompt, args.e2e_output
    config = LlamaConfig(**LLAMA32_3B, attn_implementation="sdpa")
    g = torch.Generator().manual_seed(args.seed + 99)
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=g)

    energy_uj = _energy_reader()

    def graph_request(dec):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompt)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dec.decode(O - 1)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        return t0, t1, t2

    @torch.inference_mode()
    def eager_request(model):
        # the reference's dense loop (benchmark_generation.py:74-88), fused SDPA backends only
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = model(input_ids=prompt.to(device), use_cache=True, logits_to_keep=1)
            cur, cache = out.logits[:, -1:].argmax(-1), out.past_key_values
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for _ in range(O - 1):
                out = model(input_ids=cur, past_key_values=cache, use_cache=True, logits_to_keep=1)
                cur, cache = out.logits[:, -1:].argmax(-1), out.past_key_values
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            return t0, t1, t2

    def summarize(rows, energy_total_uj):
        ttft = statistics.median((t1 - t0) * 1e3 for t0, t1, _ in rows)
        tpot = statistics.median((t2 - t1) * 1e3 / max(O - 1, 1) for _, t1, t2 in rows)
        tps = statistics.median(B * O / (t2 - t0) for t0, _, t2 in rows)
        res = {"ttft_ms": ttft, "tpot_ms": tpot, "output_tok_s": tps, "requests": len(rows)}
        if energy_total_uj is not None and energy_total_uj > 0:
            # J per 1K tokens = mJ per token (the reference's figure, benchmark_generation.py:148-155),
            # over all timed requests together: the counter updates too coarsely for one 0.5 s request
            res["energy_j_per_1k_tokens"] = energy_total_uj / 1e3 / (B * O * len(rows))
        return res

    def run(fn, target):
        for _ in range(args.e2e_warmup):
            fn(target)
        torch.cuda.synchronize()
        e0 = energy_uj()
        rows = [fn(target) for _ in range(args.e2e_repeats)]
        e1 = energy_uj()
        return summarize(rows, None if e0 is None or e1 is None else e1 - e0)

    res = {"batch": B, "prompt": P, "output": O, "keep": args.keep, "data": "random-init weights, seeded uniform "
           "prompt ids, seeded uniform tile maps"}
    t0 = time.perf_counter()
    model, stats = build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), device,
                                               keep_frac=args.keep, seed=args.seed)
    res["build_s"] = time.perf_counter() - t0
    torch.cuda.reset_peak_memory_stats()
    dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=device)
    res["tilequant_graph"] = run(graph_request, dec)
    res["tilequant_graph"]["peak_allocated_gib"] = torch.cuda.max_memory_allocated() / 2 ** 30
    res["tilequant_graph"]["decode_step"] = "fused (9 launches per layer)" if dec._fused else "model forward"
    res["tilequant_graph"]["prefill"] = "fused glue" if dec._fused_prefill else "model forward"
    dec.close()
    del dec
    if args.released_maps:
        # the same model with the released Llama-3.2-3B gi keep01 tile maps
        rmodel, _ = build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), device,
                                                keep_dir=RELEASED_MAPS / "llama32_3b_gi_keep01", seed=args.seed)
        dec = CudaGraphGreedyDecoder.prepare(rmodel, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=device)
        res["tilequant_graph_released_keep01"] = run(graph_request, dec)
        dec.close()
        del dec, rmodel
        gc.collect()
        torch.cuda.empty_cache()
    if args.e2e_module_path:
        # the reference's structure: the model's own modules replayed in the prefill and decode graphs
        dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=device,
                                             fused_decode=False, fused_prefill=False)
        res["tilequant_graph_module_step"] = run(graph_request, dec)
        dec.close()
        del dec
    del model
    gc.collect()
    torch.cuda.empty_cache()
    if not args.e2e_dense:
        return res
    dense = _dense_model(config, device, args.seed, torch.bfloat16)
    torch.cuda.reset_peak_memory_stats()
    dec = CudaGraphGreedyDecoder.prepare(dense, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=device)
    res["dense_bf16_graph"] = run(graph_request, dec)
    res["dense_bf16_graph"]["peak_allocated_gib"] = torch.cuda.max_memory_allocated() / 2 ** 30
    res["dense_bf16_graph"]["decode_step"] = "fused glue, hipBLASLt GEMMs on stacked weights" if dec._fused \
        else "model forward"
    res["dense_bf16_graph"]["prefill"] = "fused glue, hipBLASLt GEMMs on stacked weights" if dec._fused_prefill \
        else "model forward"
    dec.close()
    del dec
    if args.e2e_module_path:
        dec = CudaGraphGreedyDecoder.prepare(dense, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=device,
                                             fused_decode=False, fused_prefill=False)
        res["dense_bf16_graph_module_step"] = run(graph_request, dec)
        dec.close()
        del dec
    if args.e2e_dense_eager:
        res["dense_bf16_eager"] = run(eager_request, dense)
    del dense
    gc.collect()
    torch.cuda.empty_cache()
    tq, dg = res["tilequant_graph"], res["dense_bf16_graph"]
    res["tpot_speedup_vs_dense_graph"] = dg["tpot_ms"] / tq["tpot_ms"]
    res["ttft_speedup_vs_dense_graph"] = dg["ttft_ms"] / tq["ttft_ms"]
    if "dense_bf16_eager" in res:
        res["tpot_speedup_vs_dense_eager"] = res["dense_bf16_eager"]["tpot_ms"] / tq["tpot_ms"]
    if "dense_bf16_graph_module_step" in res:
        res["tpot_speedup_vs_dense_graph_module_step"] = res["dense_bf16_graph_module_step"]["tpot_ms"] / tq["tpot_ms"]
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args, layers, xs):
    """The reference's CPU path on a bounded sample of the same workload: the
    activation quantization with the reference's own torch ops
    (oracle/torch_ref.py = src/kernels/quant_utils.py:61-74, 103-115) and the
    mixed tile GEMM in the reference's order (oracle/tq_oracle.c, OpenMP: the
    reference has no CPU tile GEMM, so its GPU kernel's arithmetic is ported).
    Threads: the process's OMP_NUM_THREADS (16 on the GPU box) for both legs."""
    import numpy as np
    import torch
    from oracle import native as onat
    from oracle import numerics as nm
    from oracle import packing as opk
    from oracle import torch_ref

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch_threads_before = torch.get_num_threads()
    torch.set_num_threads(threads)
    onat.lib()
    work = []
    ops = 0
    for li in range(min(args.cpu_layers, len(layers))):
        for name, _, k in GROUPS:
            lin = layers[li][name]
            w8 = opk.from_mfma_int8(lin.int8_tiles.cpu().numpy())
            w16 = nm.bf16_bits_to_f32(opk.from_mfma_16bit(lin.fp16_tiles.cpu().view(torch.int16).numpy().view(np.uint16)))
            work.append(dict(x=xs[name].cpu(), w8=w8, sw=lin.int8_scales.cpu().numpy(),
                             ids8=lin.int8_tile_ids.cpu().numpy(), rp8=lin.int8_row_ptr.cpu().numpy(), w16=w16,
                             ids16=lin.fp16_tile_ids.cpu().numpy(), rp16=lin.fp16_row_ptr.cpu().numpy(),
                             n_tr=lin.n_tr, n_tc=lin.n_tc, M=lin.M_orig, K=lin.K_orig))
            ops += 2 * args.tokens * lin.M_orig * lin.K_orig
    legs = {"quant_s": 0.0, "gemm_s": 0.0}

    def run():
        for w in work:
            t0 = time.perf_counter()
            xq, sx = torch_ref.act_quant(w["x"])
            t1 = time.perf_counter()
            onat.gemm_mixed(xq.numpy(), sx.numpy(), w["x"].float().numpy(), w["w8"], w["sw"], w["ids8"], w["rp8"],
                            w["w16"], w["ids16"], w["rp16"], w["n_tr"], w["n_tc"], w["M"], w["K"])
            legs["quant_s"] += t1 - t0
            legs["gemm_s"] += time.perf_counter() - t1

    try:
        run()
        legs["quant_s"] = legs["gemm_s"] = 0.0
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or time.perf_counter() - t_start < args.cpu_seconds:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start > 30.0:
                break
    finally:
        torch_threads = torch.get_num_threads()
        torch.set_num_threads(torch_threads_before)
    t = statistics.median(times)
    reps = len(times)
    # context: the same sample as dense bf16 torch.nn.functional.linear on the same CPU threads
    dense_ms = None
    try:
        torch.set_num_threads(threads)
        g = torch.Generator().manual_seed(args.seed + 21)
        dense_w = [(w["x"], (torch.randn((w["M"], w["K"]), generator=g) * 0.02).to(torch.bfloat16)) for w in work]
        for x, wd in dense_w:
            torch.nn.functional.linear(x, wd)
        dts = []
        d_start = time.perf_counter()
        while len(dts) < 3 or (time.perf_counter() - d_start < 3.0 and len(dts) < 20):
            t0 = time.perf_counter()
            for x, wd in dense_w:
                torch.nn.functional.linear(x, wd)
            dts.append(time.perf_counter() - t0)
        dense_ms = statistics.median(dts) * 1e3
        del dense_w
    finally:
        torch.set_num_threads(torch_threads_before)
    return {"value": ops / t / 1e12, "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{min(args.cpu_layers, len(layers))} of {len(layers)} layers of the same linear set at "
                      f"{args.tokens} tokens: activation quantization with the reference's torch CPU ops "
                      "(quant_utils.py:61-74, 103-115) + tile GEMM in reference order (oracle/tq_oracle.c, "
                      f"OpenMP); median of {reps} reps over {sum(times):.1f} s, {t * 1e3:.1f} ms per sample",
            "ms_per_sample": t * 1e3,
            "quant_ms_per_sample": legs["quant_s"] / reps * 1e3, "gemm_ms_per_sample": legs["gemm_s"] / reps * 1e3,
            "host": {"cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch_threads,
                     "omp_threads": onat.num_threads()},
            "dense_bf16_cpu": None if dense_ms is None else {
                "ms_per_sample": dense_ms, "tops": ops / (dense_ms / 1e3) / 1e12,
                "note": "context: torch.nn.functional.linear in bf16 on the same sample and threads"}}


def config0_measure(args, device):
    """ONE MixedLinear 3072 -> 3072 (Llama-3.2-3B q_proj
    shape), 16 tokens, keep01 uniform (24 of 2304 tiles in bf16), activations
    N(0, 1) with 15 outlier channels x20.  GPU: the module's forward
    (activation quantization + mixed tile GEMM, as MixedLinear schedules it)
    replayed back to back in a HIP graph, HIP events on its stream, per-call
    average; the same with fresh weights per call is not needed at 9.5 MB (the
    weights stay in the Infinity Cache, as they would for a single layer
    called repeatedly).  CPU: the reference's CPU path for the same call --
    the activation quantization with its torch CPU ops (quant_utils.py:61-74,
    103-115) and the tile GEMM in its order (oracle/tq_oracle.c, OpenMP) --
    median of >= 20 calls after 3 warm-ups, on the process's threads."""
    import numpy as np
    import torch
    from oracle import native as onat
    from oracle import torch_ref
    from tilequant_amd.mixed_linear import MixedLinear
    from tilequant_amd.pack import pack_weight_from_tile_ids

    m = k = HIDDEN
    n = 16
    g = torch.Generator().manual_seed(args.seed + 100)
    W = (torch.randn((m, k), generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn((n, k), generator=g)
    x[:, torch.randperm(k, generator=g)[: round(0.005 * k)]] *= 20
    x = x.to(torch.bfloat16)
    n_tr, n_tc = m // 64, k // 64
    rng = np.random.default_rng(args.seed + 101)
    ids16 = keep_ids(n_tr, n_tc, 0.01, rng)
    ids8 = np.setdiff1d(np.arange(n_tr * n_tc), ids16)
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")
    pack = pack_weight_from_tile_ids(W.to(device), n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=cfg, tile_layout="mfma")
    lin = MixedLinear(pack, None, cfg)
    xd = x.to(device)
    reps, per_graph = 50, 100
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            lin(xd)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(per_graph):
            lin(xd)
    with torch.cuda.stream(s):
        for _ in range(3):
            graph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            graph.replay()
        e1.record(s)
    torch.cuda.synchronize()
    gpu_us = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
    ops = 2 * n * m * k
    packed = 4096 * len(ids8) + 8192 * len(ids16) + 4 * len(ids8)
    # the reference's CPU path on the same call
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    before = torch.get_num_threads()
    torch.set_num_threads(threads)
    op = None
    try:
        from oracle import numerics as nm
        from oracle import packing as opk

        op = opk.pack_weight(W.view(torch.int16).numpy().view(np.uint16), ids16)
        w16 = nm.bf16_bits_to_f32(op.fp16_tiles)

        def cpu_call():
            xq, sx = torch_ref.act_quant(x)
            return onat.gemm_mixed(xq.numpy(), sx.numpy(), x.float().numpy(), op.int8_tiles, op.int8_scales,
                                   op.int8_tile_ids, op.int8_row_ptr, w16, op.fp16_tile_ids, op.fp16_row_ptr,
                                   n_tr, n_tc, m, k)

        for _ in range(3):
            cpu_call()
        times = []
        t_start = time.perf_counter()
        while len(times) < 20 or (time.perf_counter() - t_start < 2.0 and len(times) < 2000):
            t0 = time.perf_counter()
            cpu_call()
            times.append(time.perf_counter() - t0)
        cpu_us = statistics.median(times) * 1e6
    finally:
        torch.set_num_threads(before)
    return {"shape": "3072x3072 MixedLinear, 16 tokens, keep01 uniform (24 bf16 tiles)",
            "gpu": {"us_per_call": gpu_us, "tops": ops / (gpu_us * 1e-6) / 1e12,
                    "gbps_packed_weights": packed / (gpu_us * 1e-6) / 1e9,
                    "timing": f"MixedLinear forward x {per_graph} in one HIP graph, HIP events on its stream, "
                              f"{reps} replays"},
            "cpu_reference_path": {"us_per_call": cpu_us, "tops": ops / (cpu_us * 1e-6) / 1e12, "cores": threads,
                                   "cpu_model": _cpu_model(), "reps": len(times),
                                   "path": "torch CPU activation quantization (quant_utils.py:61-74, 103-115) + "
                                           "tile GEMM in reference order (oracle/tq_oracle.c, OpenMP)"},
            "gpu_speedup": cpu_us / gpu_us, "ops": ops, "packed_weight_bytes": packed}


def released_maps_measure(args, device):
    """The released Llama-3.2-3B gi tile maps (keep01 for decode, keep05 for
    prefill) instead of seeded uniform ones: the decode linear set at
    args.tokens tokens (HIP-graph step of quant + GEMM, and GEMM launches alone
    per group) and one prefill layer at prefill_tokens.  The released maps
    cluster BF16 tiles (down_proj row tiles up to 59 of 62 in keep05)."""
    import torch
    from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax

    out = {"maps": "tests/golden/llama32_3b_gi_keep01 (decode), llama32_3b_gi_keep05 (prefill): "
                   "Decision/meta-llama_Llama-3.2-3B-Instruct/gi/tile_masks"}
    layers, info = build_layers(args, device, keep_dir=RELEASED_MAPS / "llama32_3b_gi_keep01")
    xs = make_inputs(args, device)

    def step():
        return [mods[name](xs[name]) for mods in layers for name, _, _ in GROUPS]

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g.replay()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps
    quant = {name: quantize_activation_tile_absmax(xs[name]) for name, _, _ in GROUPS}
    group_us = {}
    for gname, _, _ in GROUPS:
        items = []
        for mods in layers:
            lin = mods[gname]
            items.append((lin, torch.empty((args.tokens, lin.M_orig), device=device, dtype=torch.bfloat16)))

        def gemms():
            for lin, o in items:
                xq, sx = quant[gname]
                gemm_mixed_rows_splitk(x_fp=xs[gname], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                       int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                       int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                       fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr,
                                       M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc,
                                       out_dtype=torch.bfloat16, out=o, tile_layout=lin.tile_layout)

        s.wait_stream(torch.cuda.current_stream())   # the codes come from the default stream
        with torch.cuda.stream(s):
            gemms()
        torch.cuda.synchronize()
        gg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gg, stream=s):
            gemms()
        with torch.cuda.stream(s):
            gg.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(args.steps):
                gg.replay()
            e1.record(s)
        torch.cuda.synchronize()
        group_us[gname] = e0.elapsed_time(e1) * 1e3 / (args.steps * len(items))
        del gg
    out["decode"] = {"tokens": args.tokens, "keep": "released keep01", "ms_per_step": step_s * 1e3,
                     "tops": info["ops"] / step_s / 1e12, "gbps_packed_weights": info["packed_bytes"] / step_s / 1e9,
                     "hbm_frac_step": info["packed_bytes"] / step_s / 1e9 / HBM_PEAK_GBPS,
                     "packed_weight_bytes": info["packed_bytes"], "bf16_tiles": info["t16"],
                     "max_bf16_tiles_per_row_tile": info["max_bf16_per_row"], "gemm_group_avg_us": group_us}
    del layers, g
    torch.cuda.empty_cache()
    if args.prefill_tokens > 0:
        out["prefill"] = prefill_measure(args, device, keep_dir=RELEASED_MAPS / "llama32_3b_gi_keep05")
    return out


def decode_glue_probe(device) -> dict:
    """Per-launch graph timings of the fused decode step's glue kernels at the
    configs[4] decode shape (B = 4, hidden 3072, MLP 8192, 24 / 8 heads, 2304-key
    caches): each kernel launched 50 times (the attention once per distinct
    cache of 28) inside one HIP graph, HIP events around 20 replays, best of 3."""
    import torch
    from tilequant_amd import _native as nat
    from tilequant_amd.attention import decode_attention_workspace

    B, H, I, hq, hkv, D, L = 4, 3072, 8192, 24, 8, 128, 2304
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(0)
    s = torch.cuda.Stream()

    def per_launch_us(fn, launches):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            fn()
        best = float("inf")
        with torch.cuda.stream(s):
            for _ in range(3):
                gr.replay()
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                for _ in range(20):
                    gr.replay()
                e1.record(s)
                e1.synchronize()
                best = min(best, e0.elapsed_time(e1) * 1e3 / 20 / launches)
        torch.cuda.synchronize()
        del gr
        return round(best, 3)

    x = (torch.randn((B, H), generator=g) * 3).to(bf).to(device)
    d = (torch.randn((B, H), generator=g) * 2).to(bf).to(device)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(bf).to(device)
    h, y = torch.empty_like(x), torch.empty_like(x)
    q = torch.empty((B, H), dtype=torch.int8, device=device)
    sx = torch.empty((H // 64,), dtype=torch.float32, device=device)
    gu = (torch.randn((B, 2 * I), generator=g) * 2).to(bf).to(device)
    m = torch.empty((B, I), dtype=bf, device=device)
    mq = torch.empty((B, I), dtype=torch.int8, device=device)
    msx = torch.empty((I // 64,), dtype=torch.float32, device=device)

    def norm(delta):
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(50):
            nat.check(nat.lib().tq_add_rmsnorm_quant(
                x.data_ptr(), H, delta.data_ptr() if delta is not None else None, H, w.data_ptr(), 1e-5,
                h.data_ptr() if delta is not None else None, H, y.data_ptr(), H, q.data_ptr(), H, sx.data_ptr(), 0,
                B, H, None, st), "tq_add_rmsnorm_quant")

    def silu():
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(50):
            nat.check(nat.lib().tq_silu_mul_quant(gu.data_ptr(), 2 * I, m.data_ptr(), I, mq.data_ptr(), I,
                                                  msx.data_ptr(), 0, B, I, None, st), "tq_silu_mul_quant")

    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g).to(bf).to(device)
    cos = torch.randn((L, D), generator=g).to(bf).to(device)
    sin = torch.randn((L, D), generator=g).to(bf).to(device)
    caches = [(torch.randn((B, hkv, L, D), device=device).to(bf), torch.randn((B, hkv, L, D), device=device).to(bf))
              for _ in range(28)]
    out = torch.empty((B, hq * D), dtype=bf, device=device)
    qo = torch.empty((B, hq * D), dtype=torch.int8, device=device)
    osx = torch.empty((hq * D // 64,), dtype=torch.float32, device=device)
    pos = torch.tensor([L - 2], dtype=torch.int64, device=device)
    seq = torch.full((B,), L - 1, device=device, dtype=torch.int32)
    with torch.cuda.stream(s):
        ws = decode_attention_workspace(B, hq, L, device)

    def attention():
        st = torch.cuda.current_stream().cuda_stream
        for kc, vc in caches:
            nat.check(nat.lib().tq_decode_attention_rope(
                qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), kc.data_ptr(),
                vc.data_ptr(), kc.stride(0), kc.stride(2), kc.stride(1), seq.data_ptr(), out.data_ptr(), out.stride(0),
                D, qo.data_ptr(), qo.stride(0), osx.data_ptr(), 0, B, hq, hkv, D, L, D ** -0.5, ws.data_ptr(),
                ws.numel(), None, st), "tq_decode_attention_rope")

    return {"shape": f"B={B}, hidden {H}, MLP {I}, {hq}/{hkv} heads, {L - 1}-key caches",
            "add_rmsnorm_quant_us": per_launch_us(lambda: norm(d), 50),
            "rmsnorm_quant_no_delta_us": per_launch_us(lambda: norm(None), 50),
            "silu_mul_quant_us": per_launch_us(silu, 50),
            "attention_split_merge_quant_us": per_launch_us(attention, 28),
            "timing": "HIP events around 20 replays of one graph of the launches, best of 3; per launch"}


def attention_traffic_probe(device) -> None:
    """Three eager calls of the fused decode step's attention (RoPE form, INT8 merge) at the configs[4]
    decode shape with every key valid, then a 256 MiB elementwise copy for the counter calibration."""
    import torch
    from tilequant_amd import _native
    from tilequant_amd.attention import decode_attention_workspace

    B, hq, hkv, D, L = 4, 24, 8, 128, 2304
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g).to(torch.bfloat16).to(device)
    cos = torch.randn((L, D), generator=g).to(torch.bfloat16).to(device)
    sin = torch.randn((L, D), generator=g).to(torch.bfloat16).to(device)
    kc = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(device)
    vc = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(device)
    out = torch.empty((B, hq * D), dtype=torch.bfloat16, device=device)
    qo = torch.empty((B, hq * D), dtype=torch.int8, device=device)
    sx = torch.empty((hq * D // 64,), dtype=torch.float32, device=device)
    ws = decode_attention_workspace(B, hq, L, device)
    pos = torch.tensor([L - 1], dtype=torch.int64, device=device)
    seq = torch.full((B,), L, device=device, dtype=torch.int32)
    for _ in range(3):
        rc = _native.lib().tq_decode_attention_rope(
            qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), kc.stride(0), kc.stride(2), kc.stride(1), seq.data_ptr(), out.data_ptr(), out.stride(0),
            D, qo.data_ptr(), qo.stride(0), sx.data_ptr(), 0, B, hq, hkv, D, L, D ** -0.5, ws.data_ptr(),
            ws.numel(), None, torch.cuda.current_stream().cuda_stream)
        _native.check(rc, "tq_decode_attention_rope")
    torch.cuda.synchronize()
    src = torch.ones(TRAFFIC_COPY_BYTES // 4, device=device, dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"attention_traffic_probe": "done", "kv_bytes": 2 * B * hkv * L * D * 2,
                      "copy_bytes": TRAFFIC_COPY_BYTES}), flush=True)


def main():
    args = parse()
    if args.trace_split:
        trace_split(args.trace_split, args.layers)
        return
    if args.traffic_summarize:
        traffic_summarize(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from tilequant_amd import _native
    from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax

    _native.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.e2e_only:
        print(json.dumps({"e2e": e2e_measure(args, device)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_measure(args, device)}), flush=True)
        return
    if args.released_only:
        print(json.dumps({"released_maps": released_maps_measure(args, device)}), flush=True)
        return
    if args.qwen_only:
        print(json.dumps({"qwen": qwen_measure(args, device)}), flush=True)
        return
    if args.attention_traffic_probe:
        attention_traffic_probe(device)
        return
    if args.decode_glue_probe:
        print(json.dumps({"decode_glue": decode_glue_probe(device)}), flush=True)
        return
    layers, info = build_layers(args, device)
    xs = make_inputs(args, device)
    if args.traffic_probe:
        quant = {name: quantize_activation_tile_absmax(xs[name]) for name, _, _ in GROUPS}
        for _ in range(3):
            for mods in layers:
                for name, _, _ in GROUPS:
                    lin = mods[name]
                    xq, sx = quant[name]
                    gemm_mixed_rows_splitk(x_fp=xs[name], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                           int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                           int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                           fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr,
                                           M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc,
                                           out_dtype=torch.bfloat16, tile_layout=lin.tile_layout)
        src = torch.ones(TRAFFIC_COPY_BYTES // 4, device=device, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)   # a plain elementwise kernel: reads and writes TRAFFIC_COPY_BYTES
        torch.cuda.synchronize()
        print(json.dumps({"traffic_probe": "done", "gemm_launches": 3 * len(layers) * len(GROUPS),
                          "copy_bytes": TRAFFIC_COPY_BYTES}), flush=True)
        return

    def step():
        outs = []
        for mods in layers:
            for name, _, _ in GROUPS:
                outs.append(mods[name](xs[name]))
        return outs

    # eager warm-up, then capture one step as a HIP graph
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):   # the warm-up stream: workspaces already exist
        outs = step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps

    # eager step time (python dispatch + launches), for context
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    eager_s = (time.perf_counter() - t0) / 3

    # GEMM kernel duration: HIP events on the launch stream bracket every GEMM
    # launch of one step (activations quantized beforehand)
    quant = {name: quantize_activation_tile_absmax(xs[name]) for name, _, _ in GROUPS}
    launches = []
    for mods in layers:
        for name, _, _ in GROUPS:
            lin = mods[name]
            xq, sx = quant[name]
            launches.append((lin, name, xq, sx, torch.empty((args.tokens, lin.M_orig), device=device,
                                                            dtype=torch.bfloat16)))

    def gemm(lin, name, xq, sx, out):
        gemm_mixed_rows_splitk(x_fp=xs[name], x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                               int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                               int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                               fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr, M=lin.M_orig,
                               K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc, out_dtype=torch.bfloat16, out=out,
                               tile_layout=lin.tile_layout)

    for item in launches:
        gemm(*item)
    torch.cuda.synchronize()
    # GEMM kernel duration: the step's 112 GEMM launches (activations quantized
    # beforehand) captured back to back in one HIP graph on stream s; HIP events
    # on that stream bracket the replays, so the per-launch average covers the
    # kernels and the gaps between them, nothing else.
    with torch.cuda.stream(s):
        for item in launches:
            gemm(*item)
    torch.cuda.synchronize()
    ggraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ggraph, stream=s):
        for item in launches:
            gemm(*item)
    reps = max(3, args.steps)
    with torch.cuda.stream(s):
        for _ in range(2):
            ggraph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            ggraph.replay()
        e1.record(s)
    torch.cuda.synchronize()
    total_ms = e0.elapsed_time(e1)
    n_launch = reps * len(launches)
    # per-group durations: one graph per projection group (28 launches each)
    group_us = {}
    for gname, _, _ in GROUPS:
        sub = [item for item in launches if item[1] == gname]
        gg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gg, stream=s):
            for item in sub:
                gemm(*item)
        with torch.cuda.stream(s):
            gg.replay()
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record(s)
            for _ in range(reps):
                gg.replay()
            a1.record(s)
        torch.cuda.synchronize()
        group_us[gname] = a0.elapsed_time(a1) * 1e3 / (reps * len(sub))
        del gg
    gemm_avg_s = total_ms / n_launch / 1e3
    bytes_per_launch = info["packed_bytes"] / len(launches)
    achieved = bytes_per_launch / gemm_avg_s / 1e9
    plain_read_us = plain_read_launch_us(device, s, len(launches), int(bytes_per_launch), reps)
    group_plain_us = {}
    for gname, _, _ in GROUPS:
        lin0 = layers[0][gname]
        gbytes = 4096 * int(lin0.int8_tiles.shape[0]) + 8192 * int(lin0.fp16_tiles.shape[0]) + \
            4 * int(lin0.int8_tiles.shape[0])
        group_plain_us[gname] = plain_read_launch_us(device, s, len(layers), gbytes, reps)

    # dense bf16 context: the same linear set through torch.nn.functional.linear (hipBLASLt)
    dense = None
    if not args.no_dense:
        ws = [{name: torch.randn((sum(w), k), device=device, dtype=torch.bfloat16) * 0.02 for name, w, k in GROUPS}
              for _ in range(args.layers)]

        def dstep():
            return [torch.nn.functional.linear(xs[name], lw[name]) for lw in ws for name, _, _ in GROUPS]

        for _ in range(2):
            dstep()
        torch.cuda.synchronize()
        dg = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            dstep()
        torch.cuda.synchronize()
        with torch.cuda.graph(dg, stream=s):
            dstep()
        for _ in range(args.warmup):
            dg.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            dg.replay()
        torch.cuda.synchronize()
        d_s = (time.perf_counter() - t0) / args.steps
        dense_bytes = sum(sum(w) * k * 2 for _, w, k in GROUPS) * args.layers
        dense = {"ms_per_step": d_s * 1e3, "tops": info["ops"] / d_s / 1e12, "gbps": dense_bytes / d_s / 1e9,
                 "speedup_of_tilequant": d_s / step_s}
        del dg
        if args.m_sweep:
            # the same dense step at the M-sweep's token counts (one graph each, best of 3 x 10 replays)
            dense["ms_per_step_at"] = {}
            for m in (1, 16, 64):
                a2 = argparse.Namespace(**vars(args))
                a2.tokens = m
                xm = make_inputs(a2, device)

                def dstep_m():
                    return [torch.nn.functional.linear(xm[name], lw[name]) for lw in ws for name, _, _ in GROUPS]

                dstep_m()
                torch.cuda.synchronize()
                with torch.cuda.stream(s):
                    dstep_m()
                torch.cuda.synchronize()
                gm = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gm, stream=s):
                    dstep_m()
                best = float("inf")
                with torch.cuda.stream(s):
                    for _ in range(2):
                        gm.replay()
                    for _ in range(3):
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record(s)
                        for _ in range(10):
                            gm.replay()
                        e1.record(s)
                        e1.synchronize()
                        best = min(best, e0.elapsed_time(e1) / 10)
                torch.cuda.synchronize()
                dense["ms_per_step_at"][str(m)] = best
                del gm, xm
        del ws

    cpu = cpu_baseline(args, layers, xs) if args.cpu_layers > 0 else None
    config0 = config0_measure(args, device) if args.config0 else None
    m_sweep = decode_m_sweep(args, device, layers, info) if args.m_sweep else None
    if m_sweep and dense and "ms_per_step_at" in dense:
        for m, r in m_sweep.items():
            if m in dense["ms_per_step_at"]:
                r["dense_bf16_ms_per_step"] = dense["ms_per_step_at"][m]
                r["speedup_vs_dense_bf16"] = dense["ms_per_step_at"][m] / r["ms_per_step"]
    del layers
    prefill = prefill_measure(args, device) if args.prefill_tokens > 0 else None
    torch.cuda.empty_cache()
    released = released_maps_measure(args, device) if args.released_maps else None
    torch.cuda.empty_cache()
    qwen = qwen_measure(args, device) if args.qwen else None
    torch.cuda.empty_cache()
    e2e = e2e_measure(args, device) if args.e2e else None

    result = {
        "metric": "mixed tile GEMM TOPS + % roofline (M=4 decode, M=8192 prefill); TPOT",
        "value": info["ops"] / step_s / 1e12,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init weights and activations, uniform keep01 tile masks)",
        "config": {"workload": f"Llama-3.2-3B decoder linear set x {args.layers} layers at decode "
                               f"(BASELINE configs[1]), {args.tokens} tokens, keep{int(args.keep * 100):02d} "
                               "uniform tile mask, HIP-graph step of quant + mixed GEMM for QKV/O/GateUp/Down",
                   "tokens": args.tokens, "layers": args.layers, "keep": args.keep,
                   "packed_weight_bytes": info["packed_bytes"], "int8_tiles": info["t8"], "bf16_tiles": info["t16"],
                   "max_bf16_tiles_per_row_tile": info["max_bf16_per_row"]},
        "gbps_packed_weights": info["packed_bytes"] / step_s / 1e9,
        "hbm_frac_step": info["packed_bytes"] / step_s / 1e9 / HBM_PEAK_GBPS,
        "eager_ms_per_step": eager_s * 1e3,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic_for(args),
                     "kernel": "tq::gemm_decode_kernel", "avg_launch_us": gemm_avg_s * 1e6,
                     "bytes_per_launch": bytes_per_launch, "launches_per_step": len(launches),
                     "group_avg_us": group_us,
                     "plain_read_us": plain_read_us,
                     "frac_of_plain_read": plain_read_us / (gemm_avg_s * 1e6),
                     "group_plain_read_us": group_plain_us,
                     "group_frac_of_plain_read": {g: group_plain_us[g] / group_us[g] for g in group_us},
                     "timing": "HIP events on the launch stream around replays of one HIP graph holding the "
                               "step's 112 GEMM launches back to back (activations quantized beforehand); "
                               "per-launch average includes the inter-kernel gaps. plain_read_us: the same "
                               "protocol for 112 launches of a read-only kernel (tq_read_probe) over as many "
                               "distinct bytes each as a GEMM launch reads; frac_of_plain_read = plain / GEMM "
                               "time per launch"},
        "dense_bf16": dense,
        "config0": config0,
        "decode_m_sweep": m_sweep,
        "prefill": prefill,
        "qwen": qwen,
        "released_maps": released,
        "e2e": e2e,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
