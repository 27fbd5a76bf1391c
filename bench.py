#!/usr/bin/env python3
"""Per-frame decode benchmark on one MI355X.

Workload (default): the 28-layer 3B backbone step plus 7 sequential depth-decoder passes
(decoder: 4 layers, hidden 1024, 8q/2kv heads, head_dim 128, SwiGLU 8192, int8 codebook
heads 8197x1024), batch 8 (4 takes x CFG cond/uncond), attended KV length 750, the whole
frame (embedding, backbone, 8 heads, 8 CFG samplings, 7 decoder passes) replayed as one
hipGraph.  Random-init weights quantised to int8 per row on the GPU; KV cache prefilled
with N(0, 1) values; everything resident in HBM before the timed region.

Prints one JSON line: frames/s (value); the roofline of the dominant kernel (the backbone's
layer-tail launch: algorithmic bytes per launch over its hipEvent-timed mean launch time, the 28
launches of one frame captured and replayed on their own stream); the GEMV family of one frame
(every int8-weight launch); the same frame at a second KV length (``target_point``, default
4096, with the backbone tail's own roofline there); the prompt pass; one codec detokenize
window from codes to audio (``codec_window``); the isolated C1 kernels; the frame with the
reference's own depth decoder; and a CPU baseline: the reference's CPU path restated on torch
(``oracle/cpu_torch.py``: dequantised F.linear, SDPA, the masked decoder, the sampler) timed on
whole frames on the host cores.

    python bench.py [--steps K] [--warmup W] [--kv 750] [--target-kv 4096] [--decoder 1024|ref]
                    [--song] [--no-cpu]

HBM traffic of the backbone tail (``roofline.traffic``) comes from two rocprofv3 counter runs
of this script with a calibration copy appended (``--copy-calib-mib``), summarised by
``--pmc-summary FETCH_CSV WRITE_CSV`` into ``profiles/frame_traffic_b8_kv750.json`` (every
kernel class of the run, the backbone tail first), which the timed run reads back.  ``--trace-summary STATS_CSV`` turns a rocprofv3
``--kernel-trace --stats`` run of this script into the per-launch-class table of one frame.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "frame_traffic_b8_kv750.json")
# the counter runs whose csv files --pmc-summary reads (from the repository root, one MI355X)
PMC_BENCH = ("python3 bench.py --steps 2 --warmup 1 --no-cpu --target-kv 0 --prompt 0 "
             "--no-isolated --no-ref-decoder --codec-steps 0 --no-song --copy-calib-mib 256")
PMC_COMMANDS = [
    "cd /tmp && export TMPDIR=/tmp && cd <repo>",
    "timeout -s KILL 600 rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch "
    "-o fetch -- " + PMC_BENCH,
    "timeout -s KILL 600 rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write "
    "-o write -- " + PMC_BENCH,
    "python3 bench.py --pmc-summary gpurun_out/pmc_fetch/fetch_counter_collection.csv "
    "gpurun_out/pmc_write/write_counter_collection.csv --copy-calib-mib 256",
]
METRIC = "frames/s (3B backbone + 7 decoder passes) @ batch 8; decode-attn+GEMV HBM GB/s"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--kv", type=int, default=750, help="attended KV length of the backbone")
    ap.add_argument("--takes", type=int, default=4)
    ap.add_argument("--decoder", choices=["1024", "ref"], default="1024")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--target-kv", type=int, default=4096,
                    help="second attended KV length, timed and reported as target_point (0 skips)")
    ap.add_argument("--target-steps", type=int, default=100)
    ap.add_argument("--codec-steps", type=int, default=10,
                    help="Euler steps of the codec detokenize window leg (0 skips it)")
    ap.add_argument("--prompt", type=int, default=256,
                    help="prompt tokens of the timed prompt pass (0 skips it)")
    ap.add_argument("--no-isolated", dest="isolated", action="store_false",
                    help="skip the isolated-kernel sweep (GEMV 3072<->8192 at 1/2/4/8 rows, "
                         "attention over 512..8192 tokens at batch 1 and 8)")
    ap.add_argument("--no-ref-decoder", dest="ref_decoder", action="store_false",
                    help="skip the frame with the reference's own depth decoder")
    ap.add_argument("--no-tail", dest="tail", action="store_false",
                    help="run each layer's O / MLP / next q|k|v as separate GEMV launches instead "
                         "of one layer-tail launch")
    ap.add_argument("--tail-attn", choices=("on", "off", "backbone", "decoder"), default="on",
                    help="which stacks run the next layer's attention inside the layer-tail "
                         "launch (the others launch attention on its own)")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="append one ecd_copy_bytes of this many MiB (counter calibration)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc counter_collection.csv files and exit")
    ap.add_argument("--no-song", dest="song", action="store_false",
                    help="skip the song leg (generate() over a 256-token prompt and 3000 frames)")
    ap.add_argument("--song-frames", type=int, default=3000)
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-launch-class table of one frame from a rocprofv3 --kernel-trace "
                         "csv of this script, and exit")
    ap.add_argument("--pmc-gemm-summary", metavar="CSV",
                    help="summarise the prompt GEMM's MFMA / VALU counters of one rocprofv3 --pmc "
                         "counter_collection.csv and exit")
    return ap.parse_args()


def gemv_bytes(M, N, K, res):
    return N * K + 2 * N + 2 * M * K + 2 * M * N + (2 * M * N if res else 0)


def attn_bytes(R, Hq, Hk, HD, lens):
    return sum(Hk * ln * HD * 4 for ln in lens) + 4 * R * Hq * HD


def time_graph(calls, torch, reps=20):
    """Capture `calls` into one hipGraph, replay it `reps` times between two hipEvents on the
    stream the kernels run on, and return the mean milliseconds per launch."""
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in calls:
            f()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        for f in calls:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps / len(calls)


def is_backbone_tail(name):
    """rocprofv3 kernel name (demangled or not) of the backbone's layer-tail kernel (CD = 6: the
    frame's 28 tail launches), not its head launch (the HEAD template argument true)."""
    import re
    return bool(re.search(r"layer_tail_kernel<6, (\d+, ){5}(true|false), false, \d+(, (true|false)){0,2}>",
                          name)
                or re.search(r"layer_tail_kernelILi6E(Li\d+E){5}Lb[01]ELb0ELi\d+E", name))


def is_backbone_stack(name):
    """rocprofv3 kernel name of the backbone's layer-stack kernel (CD = 6, head_dim 128: several
    backbone layer tails per launch)."""
    import re
    return bool(re.search(r"layer_stack_kernel<6, (\d+, ){3}128, 3, ", name)
                or re.search(r"layer_stack_kernelILi6E(Li\d+E){3}Li128ELi3E", name))


def kernel_class(name):
    """Short class name of a rocprofv3 kernel name: template arguments kept, parameter list and
    return type dropped (demangled names), or the mangled name as it stands."""
    import re
    return re.sub(r"\(.*", "", name).replace("void ", "").strip()


def pmc_summary(fetch_csv, write_csv, calib_mib):
    """HBM traffic per launch from two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, KiB per
    dispatch), each scaled by what the counter reads for the calibration copy of known size
    (ecd_copy_bytes of calib_mib MiB, read once and written once): the backbone layer-tail
    launch (the roofline's traffic), and every kernel class of the run with its dispatch count,
    so each launch class of the frame has its own figure."""
    import csv

    def per_dispatch(path, counter):
        rows = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != counter:
                    continue
                e = rows.setdefault(r["Dispatch_Id"], [r["Kernel_Name"], 0.0])
                e[1] += float(r["Counter_Value"])
        return list(rows.values())

    out, factors, by_class = {}, {}, {}
    for tag, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        rows = per_dispatch(path, counter)
        # the backbone's dominant launch: its layer-stack kernel where it runs, else its tail
        tail = [v for n, v in rows if is_backbone_stack(n)] or \
            [v for n, v in rows if is_backbone_tail(n)]
        copy = [v for n, v in rows if "copy_bytes_kernel" in n]
        if not tail or not copy:
            raise SystemExit(f"{path}: no backbone layer-tail or calibration-copy dispatches with "
                             f"{counter}")
        kib_copy = copy[-1]
        factor = kib_copy / (calib_mib * 1024.0)
        factors[tag] = factor
        kib = sum(tail) / len(tail)
        out[tag] = {"counter": counter, "tail_dispatches": len(tail),
                    "kib_per_tail_launch": round(kib, 1), "calib_copy_kib": round(kib_copy, 1),
                    "calib_expected_kib": calib_mib * 1024, "factor": round(factor, 4),
                    "bytes_per_tail_launch": int(kib * 1024 / factor)}
        for n, v in rows:
            if "copy_bytes_kernel" in n:
                continue
            c = by_class.setdefault(kernel_class(n), {"fetch": [], "write": []})
            c[tag].append(v)
    out["traffic_bytes_per_launch"] = out["fetch"]["bytes_per_tail_launch"] + \
        out["write"]["bytes_per_tail_launch"]
    classes = []
    for name, c in by_class.items():
        if not c["fetch"] or not c["write"]:
            continue
        f = sum(c["fetch"]) / len(c["fetch"]) * 1024 / factors["fetch"]
        w = sum(c["write"]) / len(c["write"]) * 1024 / factors["write"]
        classes.append({"kernel": name, "dispatches": len(c["fetch"]),
                        "fetch_bytes_per_launch": int(f), "write_bytes_per_launch": int(w),
                        "traffic_bytes_per_launch": int(f + w)})
    classes.sort(key=lambda e: -e["traffic_bytes_per_launch"] * e["dispatches"])
    out["classes"] = classes
    out["workload"] = ("frame step: 28-layer 3B backbone + 7 depth-decoder passes (4 layers, 1024 "
                       "wide), batch 8, KV 750 (bench.py's default frame), plus the run's set-up "
                       "(weight synthesis and packing, the per-token tables) and its per-kernel "
                       "timing graphs and drop-in comparison")
    out["commands"] = PMC_COMMANDS
    out["note"] = ("FETCH_SIZE and WRITE_SIZE are KiB per dispatch (L2 <-> memory, Infinity Cache "
                   "hits included); each class averages every dispatch of that kernel in the run "
                   "and divides by the counter's calibration factor (its reading for the appended "
                   f"{calib_mib} MiB ecd_copy_bytes over {calib_mib} MiB).")
    return out


def pmc_gemm_summary(path):
    """Per prompt-GEMM variant (gemm_i8p_kernel, by kernel name and grid): dispatches, MFMA and
    VALU instructions per dispatch, VALU per MFMA, LDS instructions, f16 MFMA FLOP, and the
    derived MfmaUtil (MFMA-busy cycles over GPU-active cycles x SIMDs, %) and VALUBusy (%)."""
    import csv
    disp = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if "gemm_i8p_kernel" not in r["Kernel_Name"]:
                continue
            d = disp.setdefault(r["Dispatch_Id"], {"name": r["Kernel_Name"],
                                                   "grid": r.get("Grid_Size", "")})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    if not disp:
        raise SystemExit(f"{path}: no gemm_i8p_kernel dispatches")
    groups = {}
    for d in disp.values():
        groups.setdefault((d["name"], d["grid"]), []).append(d)
    out = []
    for (name, grid), ds in sorted(groups.items(), key=lambda kv: -len(kv[1])):
        def avg(c):
            v = [d[c] for d in ds if c in d]
            return sum(v) / len(v) if v else None
        mfma, valu = avg("SQ_INSTS_MFMA"), avg("SQ_INSTS_VALU")
        mops = avg("SQ_INSTS_VALU_MFMA_MOPS_F16")
        out.append({
            "kernel": name.split("(")[0], "grid": grid, "dispatches": len(ds),
            "mfma_insts": mfma, "valu_insts": valu,
            "valu_per_mfma": round(valu / mfma, 2) if mfma and valu else None,
            "lds_insts": avg("SQ_INSTS_LDS"),
            "mfma_f16_flop": mops * 512 if mops is not None else None,
            "MfmaUtil_pct": round(avg("MfmaUtil"), 2) if avg("MfmaUtil") is not None else None,
            "VALUBusy_pct": round(avg("VALUBusy"), 2) if avg("VALUBusy") is not None else None,
        })
    return out


def measure_point(torch, E, model, dev, n, kv, steps, warmup, g):
    """Allocate the caches for attended length ``kv``, capture one frame as a hipGraph, time
    ``steps`` replays, then replay the frame's GEMV-family and attention launches one by one
    between hipEvents for their per-launch rooflines."""
    P, n_frames = 64, max(kv - 64, 1)
    Lcap = P + n_frames + 2 + 256
    if kv > Lcap:
        Lcap = kv + 258
    model.alloc(n, Lcap, cfg_scale=1.5)
    B = model.B
    for blk in model.backbone.blocks:
        blk.kc[:, :, : kv].copy_(torch.randn(blk.kc[:, :, : kv].shape, generator=g, device=dev))
        blk.vc[:, :, : kv].copy_(torch.randn(blk.vc[:, :, : kv].shape, generator=g, device=dev))
    tok = torch.randint(0, E.AUDIO_VOCAB, (B, E.N_CB), generator=g, device=dev)
    static = dict(tok=tok, pos=torch.full((B, 1), kv - 1, dtype=torch.long, device=dev))
    graph, out = model._capture(static, Lcap, 1.5, 50, 1.0)
    torch.cuda.synchronize()
    # The capture's eager warm-up frame is not measured.  A gate timeout there (seen on a
    # kernel's first dispatch on a stream) is reported and the gate regions are cleared before
    # the replays (the engine's capture does so itself, with a RuntimeWarning); a timeout in the
    # replays voids the measurement below.
    if model.tail_error():
        print(f"KV {kv}: a layer-tail launch of the eager warm-up frame timed out at a gate "
              f"(error words: backbone {model.backbone.tail_error():#x}, decoder "
              f"{model.decoder.tail_error():#x}); "
              "gate regions cleared before the timed frames", file=sys.stderr, flush=True)
        model.tail_reset()

    # ------------------------------------------------ timed frames (one hipGraph per frame)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    fps = steps / dt
    ms = dt / steps * 1e3
    # a gate wait of a persistent layer-tail launch that gave up leaves its frames undefined
    if model.tail_error():
        eb, ed = model.backbone.tail_error(), model.decoder.tail_error()
        raise RuntimeError(f"KV {kv}: a layer-tail launch timed out at a gate during the timed "
                           f"frames (error words: backbone {eb:#x}, decoder {ed:#x}); the "
                           "measurement is void")

    # ------------------------------------------------ per-kernel roofline of one frame
    # Record every C-ABI launch of one eager frame step, then replay the GEMV-family and the
    # attention launches one by one between hipEvents.  Algorithmic bytes per launch follow
    # the per-unit figures: weights N*K + scales 2N + activations in/out (+ residual).
    from estudiocanciones_amd import _ffi
    calls = []
    orig_call = _ffi.call
    orig_attn = E.Stack._attention

    def rec_call(name, *a):
        calls.append((name, a))
        return orig_call(name, *a)

    attn_lens = []

    def rec_attn(st, b, q, pos, S, splits=None):
        # the engine's standalone attention: one ecd_decode_attn launch per call
        L = b.kc.shape[2]
        attn_lens.append(((pos.cpu() + 1).clamp(0, L).tolist(), q.shape[0], b.h, b.kvh, b.hd))
        return orig_attn(st, b, q, pos, S, splits)

    # a stack's layer-0 head launch runs that layer's attention: its cache lengths
    head_lens = []
    orig_head = E.layer_head

    def rec_head(x, nxt, o_next, F, *a, **kw):
        L = nxt["L"]
        head_lens.append(((nxt["pos"].cpu() + 1).clamp(0, L).tolist(), x.shape[0], nxt["Hq"],
                          nxt["Hk"], nxt["HD"]))
        return orig_head(x, nxt, o_next, F, *a, **kw)

    _ffi.call, E.Stack._attention, E.layer_head = rec_call, rec_attn, rec_head
    try:
        model._step(static["tok"], static["pos"], Lcap, 1.5, 50, 1.0)
    finally:
        _ffi.call, E.Stack._attention, E.layer_head = orig_call, orig_attn, orig_head
    torch.cuda.synchronize()

    def gemv_family_bytes(name, a):
        if name in ("ecd_gemv_i8", "ecd_gemv_i8p", "ecd_gemv_i8p_splitk"):
            # (the split-K variant's fp32 partials are workspace traffic, not algorithmic bytes)
            M, N, K = a[8], a[9], a[10]
            return N * K + 2 * N + 2 * M * K + 2 * M * N + (2 * M * N if a[4] else 0)
        if name == "ecd_rms_gemv_i8p":
            M, N, K = a[8], a[9], a[10]
            return N * K + 2 * N + 2 * M * K + 2 * K + 2 * M * N
        if name == "ecd_rms_qkv_rope":
            M, Hq, Hk, HD, K = a[11], a[13], a[14], a[16], a[17]
            N = (Hq + 2 * Hk) * HD
            return N * K + 2 * N + 2 * M * K + 2 * K + 2 * M * N + 4 * M * HD
        if name == "ecd_rms_w13_silu":
            M, F, K = a[7], a[8], a[9]
            return 2 * F * K + 4 * F + 2 * M * K + 2 * K + 2 * M * F
        if name == "ecd_layer_tail":
            # O (+res), rms -> w1|w3 -> SiLU, w2 (+res), and the next layer's rms -> q|k|v
            # (the next layer's attention, when it runs in the launch, is counted by tail_attn_bytes)
            M, D, F, Hq, Hk, HD = a[24], a[25], a[26], a[28], a[29], a[31]
            b = (D * D + 2 * D + 6 * M * D) + (2 * F * D + 4 * F + 2 * M * D + 2 * D + 2 * M * F) \
                + (D * F + 2 * D + 2 * M * F + 4 * M * D)
            if a[10]:
                Nq = (Hq + 2 * Hk) * HD
                b += Nq * D + 2 * Nq + 2 * M * D + 2 * D + 2 * M * Nq + 4 * M * HD
            return b
        if name == "ecd_layer_stack":
            # nl layer tails in one launch: every layer's O, MLP, and all but the last layer's
            # next-layer rms -> q|k|v (their attention is counted by tail_attn_bytes)
            # (and, with a codebook head in the last layer, yn = a[18] > 0: its RMS-prologue GEMV)
            nl, M, D, F, Hq, Hk, HD, yn = a[1], a[10], a[11], a[12], a[14], a[15], a[17], a[18]
            b = (D * D + 2 * D + 6 * M * D) + (2 * F * D + 4 * F + 2 * M * D + 2 * D + 2 * M * F) \
                + (D * F + 2 * D + 2 * M * F + 4 * M * D)
            Nq = (Hq + 2 * Hk) * HD
            hb = yn * D + 2 * yn + 2 * M * D + 2 * D + 2 * M * yn if yn else 0
            return nl * b + (nl - 1) * (Nq * D + 2 * Nq + 2 * M * D + 2 * D + 2 * M * Nq + 4 * M * HD) + hb
        if name == "ecd_layer_head":
            # rms -> q|k|v of layer 0 (its attention is counted by tail_attn_bytes)
            M, D, Hq, Hk, HD = a[13], a[14], a[17], a[18], a[20]
            Nq = (Hq + 2 * Hk) * HD
            return Nq * D + 2 * Nq + 2 * M * D + 2 * D + 2 * M * Nq + 4 * M * HD
        if name == "ecd_embed_gemv_i8p":
            M, N, K = a[12], a[13], a[14]
            ev = 2 * (M // 2) * K if a[7] else 0
            return N * K + 2 * N + M * K + ev + 2 * M * N
        return None

    # a layer-tail launch with o_next (argument 17) also runs the next layer's decode attention:
    # its cache lengths are those of the stack's layer-0 attention (a decode-attention launch or
    # the head launch), the latest before it
    tail_att = {}
    k_att, k_head, last = -1, -1, None
    for i, (n, a) in enumerate(calls):
        if n == "ecd_decode_attn":
            k_att += 1
            last = attn_lens[k_att]
        elif n == "ecd_layer_head":
            k_head += 1
            last = head_lens[k_head]
            lens, R, Hq, Hk, HD = last
            tail_att[i] = attn_bytes(R, Hq, Hk, HD, lens)
        elif n == "ecd_layer_tail" and a[17]:
            lens, R, Hq, Hk, HD = last
            tail_att[i] = attn_bytes(R, Hq, Hk, HD, lens)
        elif n == "ecd_layer_stack":
            lens, R, Hq, Hk, HD = last
            tail_att[i] = (a[1] - 1) * attn_bytes(R, Hq, Hk, HD, lens)
    gemv_calls = [(n, a, gemv_family_bytes(n, a) + tail_att.get(i, 0))
                  for i, (n, a) in enumerate(calls) if gemv_family_bytes(n, a)]
    attn_calls = [(n, a) for n, a in calls if n == "ecd_decode_attn"]
    assert len(attn_calls) == len(attn_lens), (len(attn_calls), len(attn_lens))
    gemv_b = [b for _, _, b in gemv_calls]
    attn_b = [sum(Hk * ln * HD * 4 for ln in lens) + 4 * R * Hq * HD for lens, R, Hq, Hk, HD in attn_lens]
    def relaunch(name, a):
        # the recorded stream handle is replaced by the stream current at replay (capture) time
        return lambda: orig_call(name, *a[:-1], torch.cuda.current_stream().cuda_stream)

    g_ms_launch = time_graph([relaunch(n, a) for n, a, _ in gemv_calls], torch)
    g_ms_total = g_ms_launch * len(gemv_calls)
    # the dominant kernel: the backbone's layer-stack launches (one call of the 28 layers, 7 per
    # kernel launch; recognised by the backbone's plan), or its layer-tail launches (recognised
    # by their O-projection weights: the reference decoder's tails are 3072 wide too)
    bb_plans = {t["plan"].data_ptr() for t in (model.backbone.tail, model.backbone.tail2)
                if t is not None and t.get("plan") is not None}
    bs = [(n, a, b) for n, a, b in gemv_calls if n == "ecd_layer_stack" and a[0] in bb_plans]
    bb_wo = {b.o.qp.data_ptr() for b in model.backbone.blocks}
    bt = bs or [(n, a, b) for n, a, b in gemv_calls if n == "ecd_layer_tail" and a[2] in bb_wo]
    # kernel launches per recorded call (a stack call of nl layers: nl / layers-per-launch)
    from estudiocanciones_amd.kernels import layer_stack_layers_per_launch as lpl
    bt_k = [1 if n == "ecd_layer_tail" else
            a[1] // lpl(a[1], a[10], a[11], a[12], a[14], a[15], a[17], a[16], bool(a[21] & 2),
                        bool(a[21] & 8))
            for n, a, _ in bt]
    bt_ms = time_graph([relaunch(n, a) for n, a, _ in bt], torch) * len(bt) / sum(bt_k) \
        if bt else None
    bt_bytes = sum(b for _, _, b in bt) / sum(bt_k) if bt else None
    bt_att = bool(bt) and (bool(bs) or bool(bt[0][1][17]))
    bt_stack = bool(bs)
    bt_lpl = bs[0][1][1] // bt_k[0] if bs else 1
    bb_idx = [i for i, b in enumerate(attn_b) if b > 10e6]
    # (no standalone attention launch is left when every layer's attention runs in a launch)
    a_ms_launch = time_graph([relaunch(*c) for c in attn_calls], torch) if attn_calls else 0.0
    a_ms_total = a_ms_launch * len(attn_calls)
    bb_ms = time_graph([relaunch(*attn_calls[i]) for i in bb_idx], torch) if bb_idx else None
    g_avg_us = g_ms_launch * 1e3
    g_bytes_avg = sum(gemv_b) / len(gemv_b)
    g_gbps = sum(gemv_b) / (g_ms_total * 1e-3) / 1e9
    a_gbps = sum(attn_b) / (a_ms_total * 1e-3) / 1e9 if attn_calls else None
    bb_attn_gbps = (sum(attn_b[i] for i in bb_idx) / (bb_ms * len(bb_idx) * 1e-3) / 1e9) if bb_idx else None
    frame_bytes = sum(gemv_b) + sum(attn_b)
    launches = len(calls)
    del graph
    return dict(Lcap=Lcap, fps=fps, ms=ms, timed_s=dt, g_gbps=g_gbps, a_gbps=a_gbps,
                bb_attn_gbps=bb_attn_gbps, gemv_b=gemv_b, attn_b=attn_b, g_avg_us=g_avg_us,
                g_bytes_avg=g_bytes_avg, g_ms_total=g_ms_total, a_ms_total=a_ms_total,
                a_ms_launch=a_ms_launch, frame_bytes=frame_bytes, launches=launches,
                bt_ms=bt_ms, bt_bytes=bt_bytes, bt_n=sum(bt_k), bt_att=bt_att, bt_stack=bt_stack,
                bt_lpl=bt_lpl)


def roofline_entry(pt, traffic):
    """The dominant kernel of the frame: the backbone's layer-tail launch (28 per frame, one
    shape).  achieved = its algorithmic bytes per launch / its mean launch time (graph replay of
    the frame's 28 launches between hipEvents on their stream)."""
    if not pt["bt_ms"]:
        return {"bound": "hbm", "kernel": "layer tail not in use", "achieved": None,
                "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": None, "traffic": None}
    ach = pt["bt_bytes"] / (pt["bt_ms"] * 1e-3) / 1e9
    what = "O + MLP + next layer's rms+q|k|v+RoPE" + (" + its decode attention"
                                                      if pt["bt_att"] else "")
    kern = (f"layer_stack_kernel, backbone width 3072, {pt['bt_lpl']} layers per launch (each "
            f"{what})" if pt.get("bt_stack") else f"layer_tail_kernel, backbone width 3072 ({what})")
    return {
        "bound": "hbm",
        "kernel": kern,
        "achieved": round(ach, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(ach / HBM_PEAK_GBPS, 4),
        "traffic": traffic,
        "traffic_source": ("rocprofv3 FETCH_SIZE + WRITE_SIZE per backbone layer-stack (or "
                           "layer-tail) dispatch, copy-calibrated "
                           "(profiles/frame_traffic_b8_kv750.json)")
                          if traffic else None,
        "avg_launch_us": round(pt["bt_ms"] * 1e3, 3),
        "algorithmic_bytes_per_launch": int(pt["bt_bytes"]),
        "launches_per_frame": pt["bt_n"],
    }


def main():
    args = parse()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, args.copy_calib_mib or 256), indent=1))
        return
    if args.pmc_gemm_summary:
        print(json.dumps(pmc_gemm_summary(args.pmc_gemm_summary), indent=1))
        return
    if args.trace_summary:
        print(trace_summary(args.trace_summary))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the decode path has no "
                          "multi-GPU mode (takes would shard by data parallelism with no collectives)"}))
        sys.exit(2)
    import torch
    from estudiocanciones_amd import engine as E
    from estudiocanciones_amd import kernels as KK
    from estudiocanciones_amd.quant import synthetic_weights

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bb = dict(E.BACKBONE, ffn=8192)
    dec = dict(E.DECODER_1024 if args.decoder == "1024" else E.DECODER, ffn=8192)
    t_build = time.time()
    w = synthetic_weights(bb, dec, dev, seed=args.seed)
    model = E.HeartMuLaLite(w, device=dev, backbone=bb, decoder=dec)
    model.backbone.use_tail = model.decoder.use_tail = args.tail
    model.backbone.tail_attention = args.tail_attn in ("on", "backbone")
    model.decoder.tail_attention = args.tail_attn in ("on", "decoder")
    wcpu = None if args.no_cpu else {k: v.cpu() for k, v in w.items()}
    del w
    n = args.takes
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 1)
    t_build = time.time() - t_build
    main_pt = measure_point(torch, E, model, dev, n, args.kv, args.steps, args.warmup, g)
    B, Lcap = model.B, main_pt["Lcap"]
    target = None
    if args.target_kv > 0 and args.target_kv != args.kv:
        tp = measure_point(torch, E, model, dev, n, args.target_kv, args.target_steps, args.warmup, g)
        target = {
            "kv_len": args.target_kv, "steps": args.target_steps,
            "value": round(tp["fps"], 2), "unit": "frames/s", "ms_per_step": round(tp["ms"], 4),
            "gemv_frac": round(tp["g_gbps"] / HBM_PEAK_GBPS, 4),
            "decode_attn_frac": (round(tp["a_gbps"] / HBM_PEAK_GBPS, 4) if tp["a_gbps"]
                                 else None),
            "backbone_attn_GBps": round(tp["bb_attn_gbps"], 1) if tp["bb_attn_gbps"] else None,
            "backbone_attn_frac": (round(tp["bb_attn_gbps"] / HBM_PEAK_GBPS, 4)
                                   if tp["bb_attn_gbps"] else None),
            "frame_frac_of_hbm": round(tp["frame_bytes"] * tp["fps"] / 1e9 / HBM_PEAK_GBPS, 4),
            "backbone_tail": roofline_entry(tp, None),
        }
    # the reference decoder's frame right after the headline points (the GPU in the same state,
    # the same number of timed steps)
    ref_dec = (measure_ref_decoder(torch, E, bb, dev, n, args, g)
               if args.ref_decoder and args.decoder == "1024" else None)
    fps, ms = main_pt["fps"], main_pt["ms"]
    g_gbps, a_gbps, bb_attn_gbps = main_pt["g_gbps"], main_pt["a_gbps"], main_pt["bb_attn_gbps"]
    gemv_b, attn_b = main_pt["gemv_b"], main_pt["attn_b"]
    g_avg_us, g_bytes_avg = main_pt["g_avg_us"], main_pt["g_bytes_avg"]
    g_ms_total, a_ms_total, a_ms_launch = main_pt["g_ms_total"], main_pt["a_ms_total"], main_pt["a_ms_launch"]
    frame_bytes, launches = main_pt["frame_bytes"], main_pt["launches"]
    from estudiocanciones_amd import _ffi
    if args.copy_calib_mib > 0:
        # calibration for the counter runs: one plain copy of known size, read once, written once
        nb = args.copy_calib_mib << 20
        src = torch.empty(nb, dtype=torch.int8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        _ffi.call("ecd_copy_bytes", src.data_ptr(), dst.data_ptr(), nb,
                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    prompt = None
    if args.prompt > 0 and args.prompt <= Lcap:
        # prompt pass (runs after the frame measurements: it overwrites cache slots [0, P))
        P = args.prompt
        xp = torch.randn(B, P, bb["dim"], generator=g, device=dev).to(torch.float16)
        pp = torch.arange(P, device=dev)[None].expand(B, P).contiguous()
        model.backbone(xp, pp)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            model.backbone(xp, pp)
        e1.record()
        torch.cuda.synchronize()
        p_ms = e0.elapsed_time(e1) / 3
        hd = bb["dim"] // bb["heads"]
        per_layer = 2 * B * P * sum(N * K for N, K in (
            ((bb["heads"] + 2 * bb["kv_heads"]) * hd, bb["dim"]), (bb["dim"], bb["dim"]),
            (2 * bb["ffn"], bb["dim"]), (bb["dim"], bb["ffn"])))
        flops = per_layer * bb["layers"]
        prompt = {"prompt_tokens": P, "rows": B * P, "ms": round(p_ms, 3),
                  "gemm_flops": int(flops), "gemm_equivalent_TFLOPs": round(flops / p_ms / 1e9, 1),
                  "frac_of_mfma_f16_peak": round(flops / p_ms / 1e9 / 2500.0, 4),
                  "path": ("MFMA GEMM (dense numerics, 2-stage LDS DMA) + MFMA causal flash "
                          "attention, 28 layers")}
    codec = measure_codec(torch, dev, args.codec_steps, args.seed) if args.codec_steps > 0 else None
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")

    res = {
        "metric": METRIC,
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: random-init weights quantised to int8 per row, N(0,1) KV cache",
        "config": {
            "workload": ("frame step: 28-layer 3B backbone (3072, 24q/8kv, hd128, FFN 8192) + "
                         + ("7 depth-decoder passes (4 layers, 1024, 8q/2kv, hd128, FFN 8192)"
                            if args.decoder == "1024" else
                            "7 depth-decoder passes (3 layers, 3072, 8q/4kv, hd384, FFN 8192)")
                         + f", int8 heads 8197, batch {B} ({n} takes x CFG), KV length {args.kv}, "
                           "whole frame as one hipGraph"),
            "batch": B, "takes": n, "kv_len": args.kv, "kv_capacity": Lcap,
        },
        "tokens_per_s": round(fps * E.N_CB * n, 1),
        "roofline": roofline_entry(main_pt, traffic),
        "gemv_family": {
            "kernels": ("every int8-weight GEMV call of one frame (C-ABI calls; a layer-stack call "
                        "counts once): layer stacks and tails, rms+q|k|v+RoPE, rms+w1|w3+SiLU, "
                        "plain / split-K GEMVs, codebook heads"),
            "achieved_GBps": round(g_gbps, 1),
            "frac": round(g_gbps / HBM_PEAK_GBPS, 4),
            "avg_launch_us": round(g_avg_us, 3),
            "algorithmic_bytes_per_launch": int(g_bytes_avg),
            "launches_per_frame": len(gemv_b),
        },
        "decode_attn": {
            "achieved_GBps": round(a_gbps, 1) if a_gbps else None,
            "frac": round(a_gbps / HBM_PEAK_GBPS, 4) if a_gbps else None,
            "backbone_layer_GBps": round(bb_attn_gbps, 1) if bb_attn_gbps else None,
            "avg_launch_us": round(a_ms_launch * 1e3, 3) if attn_b else None,
            "launches_per_frame": len(attn_b),
        },
        "frame": {
            "algorithmic_bytes": int(frame_bytes),
            "effective_GBps": round(frame_bytes * fps / 1e9, 1),
            "frac_of_hbm": round(frame_bytes * fps / 1e9 / HBM_PEAK_GBPS, 4),
            "kernel_time_gemv_ms": round(g_ms_total, 4),
            "kernel_time_attn_ms": round(a_ms_total, 4),
            "library_launches": launches,
        },
        "target_point": target,
        "prompt_pass": prompt,
        "codec_window": codec,
        "setup_s": round(t_build, 1),
    }
    if args.song:
        tp_ms = target["ms_per_step"] if target else None
        res["song"] = measure_song(torch, E, model, dev, n, args.song_frames, args.prompt or 256,
                                   (args.kv, ms), (args.target_kv, tp_ms), g)
    if args.isolated:
        res["isolated"] = measure_isolated(torch, dev)
    res["drop_in"] = measure_drop_in(torch, E, KK, model, dev, n, args.kv, g)
    del model
    torch.cuda.empty_cache()
    if ref_dec is not None:
        res["ref_decoder"] = ref_dec
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(wcpu, bb, dec, n, args.kv, args.cpu_seconds)
    print(json.dumps(res), flush=True)


def measure_song(torch, E, model, dev, n, frames, P, pt_a, pt_b, g):
    """The 4-minute song regime through HeartMuLaLite.generate (app/engine.py:374-448): a
    P-token prompt pass, then ``frames`` frames at batch 2n with every frame's tokens forced
    (random, no EOS, cond and uncond rows alike) so the song runs to its end while the attended
    KV grows from P to P + frames; CFG 1.5, graph replay with the host's EOS / error read every
    25 frames.  Reports the alloc-time per-token tables (time and bytes, built once per batch
    size), the wall time of the whole call, its frame rate, and the host loop's share: 1 - the
    GPU time the frames need (frame time interpolated linearly in KV between the two timed
    points ``pt_a``, ``pt_b`` = (kv, ms)) over the measured wall time of the frame loop."""
    import time as _t
    B = 2 * n
    # the tables are kept across allocations with the same batch size: drop them to time a
    # first allocation
    model._next_rows = model._xnext = model._next_qkv = model._onext = None
    torch.cuda.synchronize()
    t0 = _t.perf_counter()
    model.alloc(n, P + frames + 258, cfg_scale=1.5)
    torch.cuda.synchronize()
    alloc_s = _t.perf_counter() - t0
    tab_bytes = sum(t.numel() * t.element_size() for t in (model._next_rows, model._next_qkv)
                    if t is not None)
    forced = torch.randint(0, E.AUDIO_EOS, (frames + 1, B, E.N_CB), generator=g, device=dev)
    forced[:, n:] = forced[:, :n]
    text = torch.randint(0, model.text_emb.table.shape[0], (P,), generator=g, device=dev)
    marks = []
    torch.cuda.synchronize()
    t1 = _t.perf_counter()
    out = model.generate(text, 3, max_ms=frames * E.FRAME_MS, n=n, forced=forced,
                         progress=lambda a, b: marks.append(_t.perf_counter()))
    torch.cuda.synchronize()
    wall = _t.perf_counter() - t1
    if model.frames_run != frames or out[0].shape[1] != frames + 1:
        raise RuntimeError(f"song: ran {model.frames_run} of {frames} frames")
    # frames 25 .. frames - 25 between the first and last progress marks (graph replays only)
    loop_s = marks[-1] - marks[0] if len(marks) > 1 else None
    loop_frames = 25 * (len(marks) - 1)
    (ka, ma), (kb, mb) = pt_a, pt_b
    gpu_s = None
    if loop_s and ma and mb and kb != ka:
        slope = (mb - ma) / (kb - ka)
        kv = [P + 25 + i for i in range(loop_frames)]
        gpu_s = sum(ma + slope * (k - ka) for k in kv) / 1e3
    return {
        "workload": (f"generate(): {P}-token prompt, {frames} forced frames (KV {P} -> "
                     f"{P + frames}), batch {B} ({n} takes x CFG 1.5), graph replay"),
        "alloc_tables_s": round(alloc_s, 3),
        "tables_bytes": int(tab_bytes),
        "wall_s": round(wall, 3),
        "frames_per_s": round(frames / wall, 2),
        "loop_frames_per_s": round(loop_frames / loop_s, 2) if loop_s else None,
        "first_25_frames_s": round(marks[0] - t1, 4) if marks else None,
        "host_loop_share": round(1 - gpu_s / loop_s, 4) if gpu_s else None,
        "host_loop_share_basis": "frame time interpolated in KV between the timed points "
                                 f"{ka} and {kb}",
    }


def trace_summary(path, nframes=10):
    """One frame's launches by kernel from a rocprofv3 --kernel-trace csv of this script: the
    dispatches are ordered by start time, frames begin at each embed_sum launch (the frame's
    first kernel), and the table averages the last ``nframes`` complete graph-replayed frames
    before the final two: per kernel the time per frame, launches per frame and the mean launch
    time, plus the frame's span, kernel-time sum and gaps."""
    import collections
    import csv
    import re
    rows = list(csv.DictReader(open(path, newline="")))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))

    def short(name):
        n = re.sub(r"\(.*", "", name).replace("void ", "")
        return n[:90]
    starts = [i for i, r in enumerate(rows) if "embed_sum" in r["Kernel_Name"]]
    frames = [(starts[k], starts[k + 1]) for k in range(len(starts) - 1)]
    sel = frames[-(nframes + 2):-2] if len(frames) > nframes + 2 else frames
    if not sel:
        raise SystemExit(f"{path}: no complete frame (no two embed_sum launches)")
    tot, cnt = collections.defaultdict(float), collections.defaultdict(int)
    gaps = span = 0.0
    for a, b in sel:
        prev = None
        for r in rows[a:b]:
            t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            k = short(r["Kernel_Name"])
            tot[k] += (t1 - t0) / 1e3
            cnt[k] += 1
            if prev is not None:
                gaps += (t0 - prev) / 1e3
            prev = t1
        span += (int(rows[b - 1]["End_Timestamp"]) - int(rows[a]["Start_Timestamp"])) / 1e3
    n = len(sel)
    lines = [f"frames {n}: span {span / n:.1f} us, kernel sum {sum(tot.values()) / n:.1f} us, "
             f"gaps {gaps / n:.1f} us, launches {sum(cnt.values()) / n:.0f}"]
    for k, v in sorted(tot.items(), key=lambda kv: -kv[1]):
        lines.append(f"  {v / n:8.1f} us  {cnt[k] / n:5.0f} x {v / cnt[k]:7.2f} us  {k}")
    return "\n".join(lines)


def measure_codec(torch, dev, steps, seed):
    """One detokenize window of the codec, codes to audio: 372 codes x 8 quantizers -> code
    embedding -> the flow-matching estimator (24 + 6 layers, dim 1536 / 3072, 24 heads), batch 1
    doubled by CFG, 744 latent frames (29.76 s), ``steps`` Euler steps with guidance 1.25 ->
    the waveform decoder (timed separately), random-init fp16 weights, codes and noise resident
    on the GPU."""
    from estudiocanciones_amd import codec as C
    sd = C.random_state_dict(device=dev, seed=seed + 7)
    est = C.LlamaTransformer(sd, device=dev)
    del sd
    emb = C.CodeEmbedding(C.random_code_embedding_state_dict(device=dev, seed=seed + 9), device=dev)
    B, T = 1, 744
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 8)
    codes = torch.randint(0, 8192, (B, 8, T // 2), generator=g, device=dev)
    noise = torch.randn(B, T, 256, generator=g, device=dev).half()
    true_lat = torch.zeros(B, T, 256, device=dev, dtype=torch.float16)
    run = lambda: C.inference_codes(emb, est, codes, true_lat, T, 0, 1.25, steps, "other_seg",
                                    noise=noise, clamp=True)
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    out = run()
    e1.record()
    torch.cuda.synchronize()
    win_ms = e0.elapsed_time(e1)
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError("codec window produced non-finite latents")
    x = noise
    ic = true_lat
    mu = torch.randn(B, T, 512, generator=g, device=dev).half()
    tm = est.timestep_vectors(torch.tensor([0.5], device=dev))
    segs = [(x.view(T, 256), 256, B, 0), (ic.view(T, 256), 256, B, 0), (mu.view(T, 512), 512, B, B)]
    reps = 10
    e0.record()
    for _ in range(reps):
        est._run(segs, 2 * B, T, (tm[0][0], tm[1][0], tm[2][0], tm[3][0], False))
    e1.record()
    torch.cuda.synchronize()
    call_ms = e0.elapsed_time(e1) / reps
    fl = C.estimator_flops(est, 2 * B, T)
    del est, emb
    torch.cuda.empty_cache()
    # the waveform of the window: latents [1, 744, 256] -> 2 x 1,428,480 samples at 48 kHz
    dec = C.ScalarDecoder(C.random_decoder_state_dict(device=dev, seed=seed + 10), device=dev)
    wav = dec.decode(out)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(3):
        wav = dec.decode(out)
    e1.record()
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1) / 3
    if not bool(torch.isfinite(wav).all()):
        raise RuntimeError("codec decoder produced non-finite samples")
    dfl = C.decoder_flops(dec, T)
    del dec, wav
    torch.cuda.empty_cache()
    return {
        "workload": ("codec detokenize window, codes to audio: 372 x 8 codes -> ResidualVQ "
                     "embedding -> flow-matching estimator (24 + 6 LlamaTransformer layers, dim "
                     "1536 / 3072, 24 heads, hd 64 / 128), batch 1 x CFG 2, 744 latent frames "
                     f"(29.76 s), {steps} Euler steps, guidance 1.25 -> waveform decoder "
                     "(2048 -> 64 channels, x1920) -> 2 x 1,428,480 samples at 48 kHz, fp16"),
        "window_ms": round(win_ms, 2),
        "latent_frames_per_s": round(T * B / (win_ms / 1e3), 1),
        "estimator_call_ms": round(call_ms, 3),
        "estimator_flops": int(fl["total"]),
        "estimator_TFLOPs": round(fl["total"] / call_ms / 1e9, 1),
        "frac_of_mfma_f16_peak": round(fl["total"] / call_ms / 1e9 / 2500.0, 4),
        "decoder_ms": round(dec_ms, 2),
        "decoder_flops": int(dfl),
        "decoder_TFLOPs": round(dfl / dec_ms / 1e9, 1),
        "codes_to_audio_ms": round(win_ms + dec_ms, 2),
        "audio_x_realtime": round(29.76 / ((win_ms + dec_ms) / 1e3), 1),
        "path": ("code gather-sum kernel + fp16 MFMA GEMM (packed weights, fused bias / scale / "
                 "SiLU-mul epilogues), MFMA flash attention, fused gated-residual + adaLN norms, "
                 "CFG Euler kernel; waveform decoder: convs as fp16 GEMMs reading their taps "
                 "from zero-padded activations, PReLU / residual epilogues"),
    }


def _rotated_time(torch, launches, reps=10):
    """Mean milliseconds per launch of ``launches`` (one per rotated buffer set) captured into one
    hipGraph and replayed ``reps`` times between hipEvents on the capturing stream."""
    return time_graph(launches, torch, reps=reps)


def measure_isolated(torch, dev, min_bytes=768 << 20):
    """Isolated kernels at the backbone shapes (the C1 sweep).  Each point cycles through enough
    independent buffer sets (>= 16, and > 768 MB in total) that the 256 MB Infinity Cache cannot
    serve the repeated reads: GEMV 3072 -> 8192 and 8192 -> 3072 at 1/2/4/8 rows (packed weights
    with streaming loads, the engine's path, and the drop-in int8_mm on row-major weights), and
    GQA decode attention 24q / 8kv, head_dim 128, over 512 ... 8192 cached tokens at batch 1
    and 8 (every row at position L - 1), with the reference's grid (``us``: 16 splits + the
    combine launch) and with the engine's (``engine_us``: the split attention and its merge in
    one launch, attention_kb workgroups of 8 splits per (row, kv head), one workgroup per CU)."""
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd import engine as E
    from estudiocanciones_amd import kernels as KK
    out = {"gemv": [], "attention": []}
    for N, K in ((8192, 3072), (3072, 8192)):
        wb = N * K
        sets = max(16, -(-min_bytes // wb))
        ws = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev) for _ in range(sets)]
        wps = [KK.pack_i8(w) for w in ws]
        s = (torch.rand(N, device=dev) * 1e-3 + 1e-4).half()
        for M in (1, 2, 4, 8):
            x = torch.randn(M, K, device=dev).half()
            ys = [torch.empty(M, N, device=dev, dtype=torch.float16) for _ in range(sets)]
            alg = gemv_bytes(M, N, K, False)
            ms_p = _rotated_time(torch, [lambda w=wp, y=y: KK.gemv_packed(x, w, s, N, K, out=y, stream=True)
                                         for wp, y in zip(wps, ys)])
            ms_r = _rotated_time(torch, [lambda w=w: KK.int8_mm(x, w, s) for w in ws])
            out["gemv"].append({"N": N, "K": K, "M": M, "sets": sets,
                                "algorithmic_bytes": alg,
                                "packed_us": round(ms_p * 1e3, 2),
                                "packed_GBps": round(alg / ms_p / 1e6, 1),
                                "packed_frac": round(alg / ms_p / 1e6 / HBM_PEAK_GBPS, 4),
                                "int8_mm_us": round(ms_r * 1e3, 2),
                                "int8_mm_GBps": round(alg / ms_r / 1e6, 1)})
        del ws, wps
        torch.cuda.empty_cache()
    Hq, Hk, HD, ns = 24, 8, 128, 16
    for B in (1, 8):
        for L in (512, 1024, 2048, 4096, 8192):
            cache_b = 2 * B * Hk * L * HD * 2
            sets = max(16, -(-min_bytes // cache_b))
            kcs = [torch.randn(B, Hk, L, HD, device=dev).half() for _ in range(sets)]
            vcs = [torch.randn(B, Hk, L, HD, device=dev).half() for _ in range(sets)]
            q = torch.randn(B, Hq * HD, device=dev).half()
            pos = torch.full((B,), L - 1, dtype=torch.long, device=dev)
            o = torch.empty_like(q)
            pm = torch.empty(B * Hq * ns, device=dev)
            pl = torch.empty_like(pm)
            pa = torch.empty(B * Hq * ns, HD, device=dev)
            sc = 1.0 / math.sqrt(HD)

            def one(kc, vc):
                KK._attn[(B, Hk, ns)](q, kc, vc, pos, o, pm, pl, pa, 1, Hq, Hk, L, sc, HD=HD,
                                      G=Hq // Hk, NSPLIT=ns)
                KK._attn_combine[(B * Hq,)](pm, pl, pa, o, HD=HD, NSPLIT=ns)
            ms = _rotated_time(torch, [lambda kc=kc, vc=vc: one(kc, vc) for kc, vc in zip(kcs, vcs)])
            # the engine's own attention: the split attention and its merge in one launch,
            # attention_kb workgroups of 8 splits per (row, kv head)
            ekb = E.attention_kb(B, Hk, L)
            ews = torch.empty(B * Hq * ekb * (2 + HD), device=dev)
            ecnt = torch.zeros(B * Hk, device=dev, dtype=torch.int32)

            def eng(kc, vc):
                st = torch.cuda.current_stream().cuda_stream
                _ffi.call("ecd_decode_attn_merged", q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                          pos.data_ptr(), o.data_ptr(), ews.data_ptr(), ecnt.data_ptr(), B, 1,
                          Hq, Hk, L, HD, ekb, sc, st)
            ems = _rotated_time(torch, [lambda kc=kc, vc=vc: eng(kc, vc) for kc, vc in zip(kcs, vcs)])
            alg = attn_bytes(B, Hq, Hk, HD, [L] * B)
            out["attention"].append({"B": B, "L": L, "sets": sets, "algorithmic_bytes": alg,
                                     "us": round(ms * 1e3, 2),
                                     "GBps": round(alg / ms / 1e6, 1),
                                     "frac": round(alg / ms / 1e6 / HBM_PEAK_GBPS, 4),
                                     "engine_splits": 8 * ekb,
                                     "engine_us": round(ems * 1e3, 2),
                                     "engine_frac": round(alg / ems / 1e6 / HBM_PEAK_GBPS, 4)})
            del kcs, vcs
            torch.cuda.empty_cache()
    return out


def measure_drop_in(torch, E, KK, model, dev, n, kv, g):
    """The kernel-level drop-in path: the backbone step through the entry points named as in
    app/kernels.py (Stack.decode_reference: int8_mm on the row-major weights, rms, _rope_cache,
    _attn, _attn_combine, _silu_mul -- the reference's launch sequence), against the engine's
    fused step, both as one hipGraph at batch 2 n, KV ``kv``; and the reference's unchanged
    prompt-pass Linear (int8_mm at 2048 rows) on the backbone shapes."""
    model.alloc(n, kv + 258, cfg_scale=1.5)
    B = model.B
    st = model.backbone
    x = torch.randn(B, st.dim, generator=g, device=dev).half()
    pos = torch.full((B,), kv - 1, dtype=torch.long, device=dev)
    ms_ref = time_graph([lambda: st.decode_reference(x, pos, 1)], torch)
    ms_fused = time_graph([lambda: st.decode(x, pos, 1)], torch)
    blk = st.blocks[0]
    xp = torch.randn(2048, st.dim, generator=g, device=dev).half()
    mm = torch.randn(2048, blk.w2.K, generator=g, device=dev).half()
    calls = [lambda: KK.int8_mm(xp, blk.qkv.q8, blk.qkv.s8), lambda: KK.int8_mm(xp, blk.o.q8, blk.o.s8),
             lambda: KK.int8_mm(xp, blk.w13.q8, blk.w13.s8), lambda: KK.int8_mm(mm, blk.w2.q8, blk.w2.s8)]
    ms_pre = time_graph(calls, torch) * len(calls)
    fl = 2 * 2048 * sum(l.N * l.K for l in (blk.qkv, blk.o, blk.w13, blk.w2))
    return {"backbone_step_ms_reference_sequence": round(ms_ref, 4),
            "backbone_step_ms_fused": round(ms_fused, 4),
            "workload": f"28-layer backbone step, batch {B}, KV {kv}",
            "prompt_linear_ms_per_layer_int8_mm_2048_rows": round(ms_pre, 4),
            "prompt_linear_TFLOPs": round(fl / ms_pre / 1e9, 1)}


def measure_ref_decoder(torch, E, bb, dev, n, args, g):
    """The frame with the reference's own depth decoder (3 layers, 3072 wide, 8q/4kv, head_dim
    384; app/engine.py:24, :116, :161) at the benchmarked batch and KV length."""
    from estudiocanciones_amd.quant import synthetic_weights
    dec = dict(E.DECODER, ffn=8192)
    w = synthetic_weights(bb, dec, dev, seed=args.seed + 3)
    model = E.HeartMuLaLite(w, device=dev, backbone=bb, decoder=dec)
    model.backbone.use_tail = model.decoder.use_tail = args.tail
    model.backbone.tail_attention = args.tail_attn in ("on", "backbone")
    model.decoder.tail_attention = args.tail_attn in ("on", "decoder")
    del w
    pt = measure_point(torch, E, model, dev, n, args.kv, args.steps, args.warmup, g)
    del model
    torch.cuda.empty_cache()
    return {"workload": ("frame step: 28-layer 3B backbone + 7 passes of the reference depth "
                         f"decoder (3 layers, 3072, 8q/4kv, hd384, FFN 8192), batch {2 * n}, "
                         f"KV {args.kv}, one hipGraph"),
            "value": round(pt["fps"], 2), "unit": "frames/s", "ms_per_step": round(pt["ms"], 4),
            "frame_bytes": int(pt["frame_bytes"]),
            "frame_frac_of_hbm": round(pt["frame_bytes"] * pt["fps"] / 1e9 / HBM_PEAK_GBPS, 4),
            "gemv_frac": round(pt["g_gbps"] / HBM_PEAK_GBPS, 4)}


def cpu_baseline(wcpu, bb, dec, n, kv, budget_s):
    """The reference's CPU path (oracle/cpu_torch.py: dequantised F.linear, SDPA, the masked
    decoder and the sampler of app/engine.py with fast = False) on the host cores, with
    os.cpu_count() threads as the reference sets them (app/studio.py:63-64): medians of >= 5
    timed repetitions after a warm-up of (a) one 3B layer decode step at B = 2, KV 1024 and (b)
    whole frames at B = 2 n, KV ``kv``, in bf16 (the reference's CPU dtype, the reported value)
    and fp16.  ``wcpu`` holds the benchmark's own int8 weights copied to the host."""
    import statistics
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.cpu_torch import CpuTorchModel, _Stack

    ncpu = os.cpu_count() or 1
    torch.set_num_threads(ncpu)
    t_start = time.perf_counter()

    def med(fn, reps, warm=1):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    out = {"unit": "frames/s", "cores": ncpu, "kind": "port", "torch_threads": torch.get_num_threads(),
           "cpu_model": _cpu_model()}
    gen = torch.Generator().manual_seed(0)
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        # (a) config[0]: one backbone layer step, B = 2, KV 1024 (cache N(0, 1), position 1023)
        one = dict(bb, layers=1)
        st = _Stack(wcpu, "backbone", one, dt)
        st.alloc(2, 1024, dt)
        for layer in st.layers:
            layer.kc.normal_(generator=gen)
            layer.vc.normal_(generator=gen)
        x = torch.randn(2, 1, bb["dim"], generator=gen).to(dt)
        pos = torch.full((2, 1), 1023)
        mask = torch.ones(2, 1, 1, 1024, dtype=torch.bool)
        with torch.inference_mode():
            out[f"c0_layer_ms_{tag}"] = round(med(lambda: st(x, pos, 1024, mask), 7) * 1e3, 2)
        del st
        # (b) frames of the benchmarked configuration
        m = CpuTorchModel(wcpu, bb, dec, dtype=dt)
        m.alloc(n, kv + 258)
        for st_ in (m.backbone,):
            for layer in st_.layers:
                layer.kc[:, :, : kv - 1].normal_(generator=gen)
                layer.vc[:, :, : kv - 1].normal_(generator=gen)
        tok = torch.randint(0, 8197, (m.B, 8), generator=gen)
        reps = 5 if tag == "bf16" else 5
        f_s = med(lambda: m.step(tok, kv - 1, gen=gen), reps)
        out[f"frame_ms_{tag}"] = round(f_s * 1e3, 1)
        out[f"frames_per_s_{tag}"] = round(1.0 / f_s, 3)
        del m
        if time.perf_counter() - t_start > budget_s * 4:
            break
    out["value"] = out["frames_per_s_bf16"]
    out["sample"] = (f"reference CPU path restated on torch (dequantised F.linear, SDPA, masked "
                     f"decoder, sampler; oracle/cpu_torch.py) on {ncpu} host threads: whole frames "
                     f"at batch {2 * n}, KV {kv}, median of 5 after one warm-up, bf16 (value) and "
                     f"fp16; plus one 3B layer step at batch 2, KV 1024, median of 7")
    out["wall_s"] = round(time.perf_counter() - t_start, 1)
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return None


if __name__ == "__main__":
    main()
