"""Headline benchmark: ms/frame of the moondream2 SigLIP vision tower at batch 1 on one MI355X (27 blocks + post-LN,
729 tokens, bf16, random-init weights N(0, 0.02), synthetic uniform u8 pixels), as one HIP-graph replay per frame.

Prints ONE JSON line with the headline value plus:
  roofline      the dominant kernel (largest total time in the tower) timed with HIP events on its own stream:
                algorithmic FLOPs per launch / average launch time vs the 2.5 PFLOP/s dense bf16 MFMA peak
  cpu_baseline  the oracle (the reference's PyTorch bf16 path restated, torch on the host cores) on the same
                workload, a bounded number of frames
  extra         secondary workloads (skipped with --no-extra): tower batch 13 / 256 throughput (batch 256 = the
                throughput-bound tower), text decoder prefill / decode / yes-no query (bf16 and W8A8), TRecViT
                streamed / clip; the decoder and TRecViT lines carry their own CPU baselines (the oracle on the host)
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15
PEAK_HBM = 8.0e12


def vision_flops_per_frame(layers=27, T=729, D=1152, F=4304, H=16, hd=72, Kp=588):
    g = 2 * T * (D * 3 * D + D * D + 2 * D * F)
    a = 2 * 2 * H * T * T * hd
    return layers * (g + a) + 2 * T * Kp * D


# LDS ring depth of each GEMM tile config (the kernel template's last argument)
GEMM_STAGES = {0: 4, 1: 4, 2: 4, 3: 4, 4: 3, 5: 3, 6: 3, 7: 2, 8: 4, 9: 4, 10: 4, 11: 3, 12: 2, 13: 6, 14: 2,
               15: 2, 16: 3, 17: 3, 18: 2, 19: 4, 20: 4, 21: 4, 22: 4, 23: 4, 24: 3, 25: 2, 26: 4, 27: 4}
# wave grid (WGM, WGN) of the kind-0 configs that do not use 2 x 2
GEMM_WAVES = {15: (2, 4), 16: (4, 2), 17: (2, 4), 23: (1, 4), 25: (4, 2)}
# 2 x 2 tiles over two k groups of waves (8 waves)
GEMM_KH2 = {19, 20, 21, 22, 24, 26, 27}


def gemm_symbol(cfg):
    import strix_halo_maxx_amd.ops as ops
    from strix_halo_maxx_amd import _lib
    bm, bn = ops.gemm_tile(cfg)
    if _lib.load().mx_gemm_cfg_kind(cfg) == 1:
        return f"gemm_ks_kernel<{bm}, {bn}, {GEMM_STAGES[cfg]}>"
    if cfg in GEMM_KH2:
        return f"gemm_bf16_kh2_kernel<{bm}, {bn}, {GEMM_STAGES[cfg]}>"
    wgm, wgn = GEMM_WAVES.get(cfg, (2, 2))
    return f"gemm_bf16_kernel<{bm}, {bn}, {wgm}, {wgn}, {GEMM_STAGES[cfg]}>"


def op_classes(vt, img):
    """The tower's batch-1 op classes, the launches its blocks run: the attention projection with its residual and
    ln2 in one launch (mx_gemm_bf16_res_ln) where the tower fuses it, else as a partial GEMM plus the residual-
    LayerNorm kernel; fc2 as a split-K partial GEMM plus the residual-LayerNorm kernel (the next block's ln1). As
    {label: (kernel symbol, flops per launch, algorithmic HBM bytes per launch, fn(i, block))}; one eager pass keeps
    every block's real operands, and fn(i, block) relaunches op `label` of block i on them."""
    import torch
    import strix_halo_maxx_amd.ops as ops
    B = img.shape[0]
    T, D, H, hd = vt.T, vt.D, vt.H, vt.hd
    M = B * T
    blocks = vt.blocks
    saved = []
    fused_proj = vt._fuse(blocks[0]["proj"], B, "proj")
    x = vt.embed(img)
    h = ops.layernorm(x, *blocks[0]["ln1"], eps=vt.eps)
    for i, b in enumerate(blocks):
        qkv = b["qkv"](h)
        q5 = qkv.view(B, T, 3, H, hd)
        q, k, v = (q5[:, :, j].transpose(1, 2) for j in range(3))
        a = vt.attn(q, k, v).view(M, D)
        if fused_proj:
            pp = None
            x1, h2 = b["proj"].res_ln(a, x, b["ln2"], eps=vt.eps)
        else:
            pp = b["proj"].partial(a)
            x1, h2 = ops.residual_layernorm(pp, b["proj"].b, x, b["ln2"], eps=vt.eps)
        f = b["fc1"](h2, gelu=True)
        pf = b["fc2"].partial(f)
        nxt = blocks[i + 1]["ln1"] if i + 1 < len(blocks) else vt.post_ln
        x2, hn = ops.residual_layernorm(pf, b["fc2"].b, x1, nxt, eps=vt.eps)
        saved.append((x, h, (q, k, v), a, pp, x1, h2, f, pf, nxt))
        x, h = x2, hn
    outs = {n: torch.empty(M, w, device=x.device, dtype=torch.bfloat16)
            for n, w in (("h", D), ("qkv", 3 * D), ("x", D), ("f", blocks[0]["fc1"].N))}
    a_out = torch.empty(B, T, D, device=x.device, dtype=torch.bfloat16)
    pp_out = None if fused_proj else torch.empty_like(saved[0][4])
    pf_out = torch.empty_like(saved[0][8])

    def sym(l):
        cfg = l.cfgs.get(M) or ops._TUNED.get((M, l.N, l.Kw))
        return gemm_symbol(cfg[0])

    def psym(l):
        cfg, sp = ops._TUNED_P[(M, l.N, l.Kw)]
        return f"{gemm_symbol(cfg)} x{sp} splits"
    attn_sym = ops.sdpa_symbol(B, H, T, hd)
    F, Kw2 = blocks[0]["fc1"].N, blocks[0]["fc2"].Kw
    sp_proj, sp_fc2 = (0 if fused_proj else saved[0][4].shape[0]), saved[0][8].shape[0]
    # algorithmic HBM bytes per launch: every operand once (bf16 activations / weights, fp32 split-K partials)
    classes = {
        "qkv": (sym(blocks[0]["qkv"]), 2 * M * D * 3 * D, 2 * (M * D + 3 * D * D + M * 3 * D),
                lambda i, b: b["qkv"](saved[i][1], out=outs["qkv"])),
        "attn": (attn_sym, 4 * B * H * T * T * hd, 8 * M * D, lambda i, b: ops.sdpa(*saved[i][2], out=a_out)),
    }
    if fused_proj:  # a, W, the residual in; x' and ln2(x') out
        classes["proj"] = ("gemm_rln_kernel<64, 64, 4, 1>", 2 * M * D * D, 2 * (M * D + D * D + 3 * M * D),
                           lambda i, b: b["proj"].res_ln(saved[i][3], saved[i][0], b["ln2"], eps=vt.eps,
                                                         x_out=outs["x"], y_out=outs["h"]))
    else:
        classes["proj"] = (psym(blocks[0]["proj"]), 2 * M * D * D, 2 * (M * D + D * D) + 4 * sp_proj * M * D,
                           lambda i, b: b["proj"].partial(saved[i][3], out=pp_out))
        classes["res_ln2"] = ("residual_layernorm_kernel<3>", 0, (4 * sp_proj + 6) * M * D,
                              lambda i, b: ops.residual_layernorm(saved[i][4], b["proj"].b, saved[i][0], b["ln2"],
                                                                  eps=vt.eps, x_out=outs["x"], y_out=outs["h"]))
    classes.update({
        "fc1": (sym(blocks[0]["fc1"]), 2 * M * D * F, 2 * (M * D + F * D + M * F),
                lambda i, b: b["fc1"](saved[i][6], gelu=True, out=outs["f"])),
        "fc2": (psym(blocks[0]["fc2"]), 2 * M * blocks[0]["fc2"].K * D, 2 * (M * F + D * Kw2) + 4 * sp_fc2 * M * D,
                lambda i, b: b["fc2"].partial(saved[i][7], out=pf_out)),
        "res_ln1": ("residual_layernorm_kernel<3>", 0, (4 * sp_fc2 + 6) * M * D, lambda i, b: ops.residual_layernorm(
            saved[i][8], b["fc2"].b, saved[i][5], saved[i][9], eps=vt.eps, x_out=outs["x"], y_out=outs["h"])),
    })
    return classes


def op_timing(vt, img, reps=5):
    """Per-kernel launch time inside the tower: for each op class of op_classes a HIP graph of its 27 launches (each
    on its own block's weights and activations, as in the tower) is replayed `reps` times between two HIP events
    recorded on the stream the kernels run on. Returns {label: [total_ms, launches, flops_per_launch, symbol]}."""
    import torch
    classes = op_classes(vt, img)
    blocks = vt.blocks
    res = {}
    for name, (ksym, fl, _, fn) in classes.items():
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i, b in enumerate(blocks):
                fn(i, b)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        n = reps * len(blocks)
        res[name] = [e0.elapsed_time(e1), n, fl, ksym]
        del g
    return res


def traffic_probe(vt, img, reps=3):
    """Eager launches for HBM-traffic counters (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, on this mode): after two
    passes of the tower and the eager pass that keeps every block's operands, a marker fill of 12345 floats, then each
    op class of the tower's batch-1 path
    launched `reps` x 27 times on its own blocks' operands (the op_timing classes, in order), then a marker fill of
    23456 floats and the calibration: `reps` device copies of 256 MiB (known traffic: 256 MiB read + 256 MiB
    written each). Traffic per launch = counter per dispatch x (256 MiB / the counter of one calibration copy)."""
    import torch
    vt(img)
    vt(img)
    classes = op_classes(vt, img)
    torch.cuda.synchronize()
    torch.full((12345,), 1.0, device=img.device)
    for name, (ksym, fl, _, fn) in classes.items():
        for _ in range(reps):
            for i, b in enumerate(vt.blocks):
                fn(i, b)
        torch.cuda.synchronize()
    torch.full((23456,), 1.0, device=img.device)
    src = torch.empty(256 << 20, dtype=torch.uint8, device=img.device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("[bench] traffic probe done: " + ", ".join(f"{k}={v[0]}" for k, v in classes.items()), flush=True)


def _decoder_for_probe():
    import torch
    import strix_halo_maxx_amd.md2text as mt
    import strix_halo_maxx_amd.synth as S
    dev = torch.device("cuda:0")
    dec = mt.TextDecoder(S.text_weights(0), device=dev, ctx=1024)
    img = S.activations(3, (729, 2048), "img").to(dev)
    return dec, img, S.prompt_ids(4, 64)


def decode_step_bytes(pos):
    """Algorithmic bytes of one bf16 decode step at position pos: every text weight and the LM head once, and the
    K / V cache rows 0 .. pos - 1 of every layer (decode_bench's count, at the step's own position)."""
    import strix_halo_maxx_amd.synth as S
    c = S.TXT
    D, F, L, V = c["dim"], c["ff"], c["layers"], c["vocab"]
    return 2 * L * (3 * D * D + D * D + 2 * D * F) + 2 * V * D + 2 * 2 * L * pos * D


def traffic_probe_decode(reps=3):
    """Eager bf16 decode steps for HBM-traffic counters (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE): prefill of
    730 + 64 tokens and a few warm-up steps, a marker fill of 34567 floats, `reps` one-launch decode steps
    (mx_decode_step_mk), a marker fill of 45678 floats, then `reps` device copies of 256 MiB for the calibration."""
    import torch
    dec, img, prompt = _decoder_for_probe()
    if not dec.use_mk:
        raise RuntimeError("the one-launch decode step is not in use on this device")
    dec.generate(img, prompt, 4)
    dec.prefill(img, prompt)
    dec.start_decode()
    for _ in range(2):
        dec.decode_step()
    torch.cuda.synchronize()
    torch.full((34567,), 1.0, device=img.device)
    for _ in range(reps):
        dec.decode_step()
    torch.cuda.synchronize()
    torch.full((45678,), 1.0, device=img.device)
    src = torch.empty(256 << 20, dtype=torch.uint8, device=img.device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    if dec.mk_error():
        raise RuntimeError(f"one-launch decode step reported error {dec.mk_error()}")
    print(f"[bench] decode traffic probe done: {reps} steps from position {dec.pos_base + 2}", flush=True)


def summarize_traffic_decode(fetch_csv, write_csv, reps=3):
    """Markdown summary of the two --pmc passes over `bench.py --traffic-probe-decode`: the decode steps sit between
    the run's last two marker fills, the calibration copies follow the second."""
    import strix_halo_maxx_amd.synth as S
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        seq = _pmc_sequence(path, counter)
        fills = [i for i, (k, _) in enumerate(seq) if "FillFunctor" in k]
        m0, m1 = fills[-2], fills[-1]
        probe, calib = seq[m0 + 1:m1], seq[m1 + 1:]
        copies = [v for k, v in calib if "copyBuffer" in k][:reps]  # the first ones: a small read-back follows
        if len(probe) != reps or len(copies) < reps or any("decode_mk_kernel" not in k for k, _ in probe):
            raise RuntimeError(f"{counter}: probe dispatches {[k for k, _ in probe]}, {len(copies)} calibration")
        out[counter] = ([v for _, v in probe], copies)
    fcal, wcal = (sum(out[c][1]) / reps for c in ("FETCH_SIZE", "WRITE_SIZE"))
    copy_b = 256 << 20
    ff, wf = copy_b / (fcal * 1024), copy_b / (wcal * 1024)
    pos0 = 1 + 729 + 64 + 2  # prefix + prompt, then the two warm-up steps
    rows = []
    for i in range(reps):
        fk, wk = out["FETCH_SIZE"][0][i], out["WRITE_SIZE"][0][i]
        rd, wr = fk * 1024 * ff, wk * 1024 * wf
        algo = decode_step_bytes(pos0 + i)
        rows.append(f"| {i} | {pos0 + i} | {fk:,.1f} | {wk:,.1f} | {rd / 1e6:,.1f} | {wr / 1e6:,.2f} | "
                    f"{(rd + wr) / 1e6:,.1f} | {algo / 1e6:,.1f} | {(rd + wr) / algo:.3f} |")
    head = ["| step | position | FETCH_SIZE KiB | WRITE_SIZE KiB | read MB | written MB | traffic MB | algorithmic MB | "
            "ratio |", "|---|---|---|---|---|---|---|---|---|"]
    mid = reps // 2
    fk, wk = out["FETCH_SIZE"][0][mid], out["WRITE_SIZE"][0][mid]
    blob = {"kernel": "decode_mk_kernel", "position": pos0 + mid, "bytes_per_launch": int(fk * 1024 * ff + wk * 1024 * wf),
            "algorithmic_bytes": decode_step_bytes(pos0 + mid)}
    return (f"Calibration (plain copy of 256 MiB = {copy_b:,} B read + the same written): FETCH_SIZE reads "
            f"{fcal:,.1f} KiB per copy, WRITE_SIZE {wcal:,.1f} KiB. Bytes = FETCH_SIZE x 1024 x {ff:.4f} + "
            f"WRITE_SIZE x 1024 x {wf:.4f}.\n\n" + "\n".join(head + rows) +
            "\n\nbench.py reads the JSON block below (`traffic` of the decode roofline):\n\n```json\n" +
            json.dumps(blob, indent=1) + "\n```\n")


def _pmc_sequence(path, counter):
    """[(kernel name, counter value)] per dispatch, in dispatch order, from a rocprofv3 counter_collection CSV."""
    import csv
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            d = int(r["Dispatch_Id"])
            k, v = per.get(d, (r["Kernel_Name"], 0.0))
            per[d] = (k, v + float(r["Counter_Value"]))
    return [per[d] for d in sorted(per)]


def summarize_traffic(fetch_csv, write_csv, reps=3):
    """Markdown summary (with the JSON block measured_traffic reads) of the two rocprofv3 --pmc passes (FETCH_SIZE,
    WRITE_SIZE) over `bench.py --traffic-probe`: the op-class dispatches sit between the run's last two marker fills,
    the calibration copies follow the second."""
    import torch
    import strix_halo_maxx_amd.md2 as md2
    import strix_halo_maxx_amd.synth as S
    vt = md2.VisionTower(S.vision_weights(0), device=torch.device("cuda:0"))
    img = S.images_u8(1, 1).to("cuda:0")
    with torch.inference_mode():
        vt(img)
        classes = op_classes(vt, img)
    nblk = len(vt.blocks)
    per = reps * nblk
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        seq = _pmc_sequence(path, counter)
        fills = [i for i, (k, _) in enumerate(seq) if "FillFunctor" in k]
        m0, m1 = fills[-2], fills[-1]
        probe, calib = seq[m0 + 1:m1], seq[m1 + 1:]
        if len(probe) != per * len(classes) or len(calib) < reps:
            raise RuntimeError(f"{counter}: {len(probe)} probe dispatches, {len(calib)} calibration dispatches")
        out[counter] = (probe, [v for _, v in calib[-reps:]])
    fcal, wcal = (sum(out[c][1]) / reps for c in ("FETCH_SIZE", "WRITE_SIZE"))
    copy_b = 256 << 20
    ff, wf = copy_b / (fcal * 1024), copy_b / (wcal * 1024)
    blob = {"calibration": {"copy_bytes_each_way": copy_b, "fetch_kib": round(fcal, 1), "write_kib": round(wcal, 1),
                            "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}, "ops": {}}
    rows = []
    for j, (label, (ksym, fl, algo, _)) in enumerate(classes.items()):
        fk = [v for _, v in out["FETCH_SIZE"][0][j * per:(j + 1) * per]]
        wk = [v for _, v in out["WRITE_SIZE"][0][j * per:(j + 1) * per]]
        names = {k for k, _ in out["FETCH_SIZE"][0][j * per:(j + 1) * per]}
        symbol = ksym.split(" x")[0]
        base = symbol.split("<")[0]
        if len(names) != 1 or base not in next(iter(names)):
            raise RuntimeError(f"{label}: dispatches {names} do not match {symbol}")
        fkib, wkib = sum(fk) / per, sum(wk) / per
        tb = int(fkib * 1024 * ff + wkib * 1024 * wf)
        blob["ops"][label] = {"kernel": ksym, "symbol": symbol, "fetch_kib": round(fkib, 1),
                              "write_kib": round(wkib, 1), "bytes_per_launch": tb, "algorithmic_bytes": algo}
        rows.append(f"| {label} | `{ksym}` | {fkib:,.1f} | {wkib:,.1f} | {fkib * 1024 * ff / 1e6:.2f} | "
                    f"{wkib * 1024 * wf / 1e6:.2f} | {tb / 1e6:.2f} | {algo / 1e6:.2f} | {tb / algo:.2f} |")
    head = ["| op | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | read MB | written MB | traffic MB | algorithmic MB | ratio |",
            "|---|---|---|---|---|---|---|---|---|"]
    return (f"Calibration (plain copy of 256 MiB = {copy_b:,} B read + the same written): FETCH_SIZE reads "
            f"{fcal:,.1f} KiB per copy, WRITE_SIZE {wcal:,.1f} KiB. Bytes = FETCH_SIZE x 1024 x {ff:.4f} + "
            f"WRITE_SIZE x 1024 x {wf:.4f}.\n\n" + "\n".join(head + rows) +
            "\n\nbench.py reads the JSON block below (`traffic` of the roofline line, when its dominant op ran the same "
            "kernel):\n\n```json\n" + json.dumps(blob, indent=1) + "\n```\n")


def summarize_counters(paths, reps=3):
    """Markdown table of per-op rocprofv3 --pmc counters over `bench.py --traffic-probe` (the probe dispatches sit
    between the run's last two marker fills, `reps` x 27 per op class, in op_classes order): MfmaUtil (percent of the
    active cycles the MFMA units were busy), fractions of the wave time (SQ_WAVE_CYCLES) spent waiting (s_waitcnt /
    barriers), stalled at issue, and issuing VALU / LDS / VMEM instructions, LDS bank-conflict cycles per launch, and
    the L2 hit rate, for whichever of these counters the CSVs hold (several passes: one CSV each). When a CSV holds a
    counter another one also holds, the later CSV's value is used."""
    import csv
    import torch
    import strix_halo_maxx_amd.md2 as md2
    import strix_halo_maxx_amd.synth as S
    vt = md2.VisionTower(S.vision_weights(0), device=torch.device("cuda:0"))
    img = S.images_u8(1, 1).to("cuda:0")
    with torch.inference_mode():
        vt(img)
        classes = op_classes(vt, img)
    per = reps * len(vt.blocks)
    vals = {}
    for path in paths:
        with open(path) as f:
            names = {r["Counter_Name"] for r in csv.DictReader(f)}
        for counter in sorted(names):
            seq = _pmc_sequence(path, counter)
            if counter == "MfmaUtil":  # a percentage: the mean over the dimension rows, not their sum
                rows = {}
                with open(path) as f:
                    for r in csv.DictReader(f):
                        if r["Counter_Name"] == counter:
                            rows.setdefault(int(r["Dispatch_Id"]), []).append(float(r["Counter_Value"]))
                seq = [(k, sum(rows[d]) / len(rows[d])) for (k, _), d in zip(seq, sorted(rows))]
            fills = [i for i, (k, _) in enumerate(seq) if "FillFunctor" in k]
            probe = seq[fills[-2] + 1:fills[-1]]
            if len(probe) != per * len(classes):
                raise RuntimeError(f"{counter}: {len(probe)} probe dispatches")
            vals[counter] = [sum(v for _, v in probe[j * per:(j + 1) * per]) / per for j in range(len(classes))]
    cols = []
    g = lambda c, j: vals[c][j] if c in vals else None
    if "MfmaUtil" in vals:
        cols.append(("MfmaUtil %", lambda j: f"{g('MfmaUtil', j):.1f}"))
    if "SQ_WAVE_CYCLES" in vals:
        for c, lab in (("SQ_WAIT_ANY", "waiting (waitcnt, barrier) / wave time"),
                       ("SQ_WAIT_INST_ANY", "issue-stalled / wave time"),
                       ("SQ_WAIT_INST_LDS", "LDS-issue-stalled / wave time"),
                       ("SQ_ACTIVE_INST_VALU", "VALU + MFMA issue / wave time"),
                       ("SQ_ACTIVE_INST_LDS", "LDS issue / wave time"),
                       ("SQ_INST_CYCLES_VMEM_RD", "VMEM-read issue / wave time")):
            if c in vals:
                cols.append((lab, lambda j, c=c: f"{g(c, j) / g('SQ_WAVE_CYCLES', j):.2f}"))
    if "SQ_LDS_BANK_CONFLICT" in vals:
        cols.append(("LDS bank-conflict cycles", lambda j: f"{g('SQ_LDS_BANK_CONFLICT', j):,.0f}"))
    if "TCC_HIT_sum" in vals and "TCC_MISS_sum" in vals:
        cols.append(("L2 hit rate", lambda j: f"{g('TCC_HIT_sum', j) / (g('TCC_HIT_sum', j) + g('TCC_MISS_sum', j)):.2f}"))
    head = "| op | kernel | " + " | ".join(c for c, _ in cols) + " |"
    rows = [head, "|" + "---|" * (len(cols) + 2)]
    for j, (label, (ksym, _, _, _)) in enumerate(classes.items()):
        rows.append(f"| {label} | `{ksym}` | " + " | ".join(fn(j) for _, fn in cols) + " |")
    return "\n".join(rows) + "\n"


def summarize_trace(trace_csv, top=30):
    """Kernel-trace rows grouped by (kernel, workgroups x threads per workgroup): calls, mean / median / total
    duration. Workgroups count the whole (X, Y, Z) grid."""
    import csv
    groups = {}
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            k = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "")
            k = k[:k.index("(")] if "(" in k and "<" not in k[:k.index("(")] else k[:k.rfind(">") + 1] if ">" in k else k
            wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
            nwg = 1
            for ax in "XYZ":
                nwg *= int(r[f"Grid_Size_{ax}"]) // int(r[f"Workgroup_Size_{ax}"])
            key = (k[:58], nwg, wg)
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'kernel':58s} {'workgroups':>12s} {'calls':>6s} {'mean_us':>9s} {'median_us':>9s} {'total_ms':>9s}"]
    for (k, g, wg), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
        d.sort()
        lines.append(f"{k:58s} {f'{g}x{wg}':>12s} {len(d):6d} {sum(d) / len(d):9.2f} {d[len(d) // 2]:9.2f} "
                     f"{sum(d) / 1e3:9.2f}")
    return "\n".join(lines)


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "vision_tower_b1_hbm_traffic.md")
DECODE_TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                   "decode_megakernel_hbm_traffic.md")


def measured_decode_traffic():
    """(HBM bytes per one-launch decode step, algorithmic bytes at the same position) from the committed summary of
    the decode traffic probe, or None."""
    try:
        txt = open(DECODE_TRAFFIC_FILE).read()
        blob = json.loads(txt.split("```json", 1)[1].split("```", 1)[0])
        return int(blob["bytes_per_launch"]), int(blob["algorithmic_bytes"])
    except (OSError, IndexError, ValueError, KeyError):
        return None


def measured_traffic(label, sym):
    """HBM bytes per launch of op `label` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (the JSON
    block of profiles/vision_tower_b1_hbm_traffic.md), if it was measured on the same kernel; else (None, reason)."""
    try:
        txt = open(TRAFFIC_FILE).read()
        blob = json.loads(txt.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return None, "no committed traffic summary"
    e = blob.get("ops", {}).get(label)
    if not e:
        return None, f"op {label} not in the committed traffic summary"
    if e.get("kernel") != sym:
        return None, f"committed summary measured {e.get('kernel')}, this run picked {sym}"
    return int(e["bytes_per_launch"]), os.path.relpath(TRAFFIC_FILE, os.path.dirname(TRAFFIC_FILE) + "/..")


def _cpu_threads():
    """Threads for the CPU baselines: the host's logical CPUs, at most 16 (the CPU share of one GPU on an 8-GPU host)."""
    return min(os.cpu_count() or 1, 16)


def cpu_baseline(budget_s=20.0):
    """The oracle (torch bf16 on the host cores) on the same workload: whole 27-block tower, batch 1."""
    import torch
    import oracle.md2_vision as ov
    import strix_halo_maxx_amd.synth as S
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    w = S.vision_weights(0)
    img = S.images_u8(1, 1)
    with torch.inference_mode():
        t0 = time.perf_counter()
        ov.tower(w, img)
        first = time.perf_counter() - t0
        n = max(2, min(10, int(budget_s / max(first, 1e-3))))
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            ov.tower(w, img)
            ts.append(time.perf_counter() - t0)
    return {"value": round(statistics.median(ts) * 1e3, 2), "unit": "ms/frame", "cores": threads, "kind": "port",
            "threads": threads, "host_logical_cpus": os.cpu_count(),
            "sample": f"oracle (reference's torch bf16 path restated) full 27-block tower + post-LN, batch 1, "
                      f"median of {n} frames after 1 warm-up, torch.set_num_threads({threads})"}


def block_bench(reps=200, cpu=True):
    """One SigLIP block (729 tokens x 1152, 16 heads x 72, MLP 4304, GELU-tanh, residuals; weights N(0, 0.02),
    activations N(0, 1)): the GPU block (ln1 -> qkv -> attention -> proj + residual + ln2 -> fc1 + GELU -> fc2 +
    residual, the tower's own kernels) as one HIP graph replayed `reps` times between two HIP events on its stream,
    and the oracle's block (the reference's torch bf16 block restated) on the host cores, median of 5 after 2
    warm-ups."""
    import torch
    import oracle.md2_vision as ov
    import strix_halo_maxx_amd.md2 as md2
    import strix_halo_maxx_amd.synth as S
    w = S.vision_weights(0, layers=1)
    x_cpu = S.activations(11, (729, 1152), "x")
    dev = torch.device("cuda:0")
    vt = md2.VisionTower(w, device=dev)
    b = vt.blocks[0]
    x = x_cpu.to(dev)
    for _ in range(3):
        vt.block(b, x, 1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        vt.block(b, x, 1)
    st = torch.cuda.current_stream()
    for _ in range(5):
        g.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    e1.synchronize()
    if vt.rln_error():
        raise RuntimeError(f"fused residual-LayerNorm GEMM reported error {vt.rln_error()}")
    us = e0.elapsed_time(e1) * 1e3 / reps
    fl = vision_flops_per_frame(layers=1, Kp=0)
    out = {"us_per_block": round(us, 2), "tflops": round(fl / us / 1e6, 1), "mfma_frac": round(fl / us / 1e6 / (PEAK_BF16 / 1e12), 4),
           "gflop_per_block": round(fl / 1e9, 3),
           "workload": "one SigLIP block, 729 tokens x 1152, bf16, batch 1, one HIP graph per block"}
    if cpu:
        threads = _cpu_threads()
        torch.set_num_threads(threads)
        xb = x_cpu[None]
        with torch.inference_mode():
            for _ in range(2):
                ov.block(w, 0, xb)
            ts = []
            for _ in range(5):
                t0 = time.perf_counter()
                ov.block(w, 0, xb)
                ts.append(time.perf_counter() - t0)
        out["cpu_baseline"] = {"value": round(statistics.median(ts) * 1e3, 2), "unit": "ms/block", "cores": threads,
                               "kind": "port", "threads": threads, "host_logical_cpus": os.cpu_count(),
                               "sample": f"oracle block (md2fast.py:153-157 restated), 729 tokens, median of 5 after "
                                         f"2 warm-ups, torch.set_num_threads({threads})"}
    return out


def cpu_baseline_decoder(n_tokens=8):
    """Config 2 on the host cores: the oracle decoder (the reference's torch bf16 text path restated), prefill of
    1 + 729 image tokens + 64 prompt ids once, then n_tokens greedy steps; tok/s over the decode steps."""
    import torch
    import oracle.md2_text as ot
    import strix_halo_maxx_amd.synth as S
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    w = S.text_weights(0)
    img = S.activations(3, (729, 2048), "img")
    prompt = S.prompt_ids(4, 64)
    with torch.inference_mode():
        m = ot.Text(w, 1024, S.freqs_cis(32, 2048))
        t0 = time.perf_counter()
        lg = m.prefill(img, prompt)
        t_pre = time.perf_counter() - t0
        ts = []
        for _ in range(n_tokens):
            tok = int(torch.argmax(lg))
            t0 = time.perf_counter()
            lg = m.step(tok)
            ts.append(time.perf_counter() - t0)
    med = statistics.median(ts)
    return {"value": round(1.0 / med, 2), "unit": "tok/s", "prefill_ms": round(t_pre * 1e3, 1), "cores": threads,
            "kind": "port", "threads": threads, "host_logical_cpus": os.cpu_count(),
            "sample": f"oracle text decoder, 24 layers: one prefill of 730 + 64 tokens, then {n_tokens} greedy steps "
                      f"(tok/s = 1 / median step time), torch.set_num_threads({threads})"}


def cpu_baseline_trecvit(frames=8):
    """Config 3 on the host cores: the oracle TRecViT (the reference's torch bf16 block restated), 12 blocks, 1024
    patch + 256 query tokens, `frames` streamed frames after one warm-up frame; ms/frame (median)."""
    import torch
    import oracle.trecvit as otr
    import strix_halo_maxx_amd.synth as S
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    m = otr.Model(S.trecvit_weights(0))
    fr = S.frames_u8(1, frames + 1)
    q = S.query_points(5, 256)
    qf = (q[:, 1:] / 256.0).to(torch.bfloat16)
    ts = []
    with torch.inference_mode():
        for t in range(frames + 1):
            t0 = time.perf_counter()
            m.step(fr[t], qf)
            if t:
                ts.append(time.perf_counter() - t0)
    return {"value": round(statistics.median(ts) * 1e3, 1), "unit": "ms/frame", "cores": threads, "kind": "port",
            "threads": threads, "host_logical_cpus": os.cpu_count(),
            "sample": f"oracle TRecViT, 12 blocks, 1280 tokens, median of {frames} streamed frames after 1 warm-up "
                      f"frame, torch.set_num_threads({threads}); the reference published 710.5 ms/frame at 1,072 "
                      f"tokens with 8 threads on its own CPU"}


def decode_bench(steps_tokens=128, w8a8=False):
    """Config 2: prefill (1 + 729 image tokens mask-free, then 64 prompt ids) + greedy decode on one HIP graph per
    step. Returns prefill ms, decode tok/s and the decode step's HBM roofline (algorithmic bytes = every weight once
    + the KV cache read per token). w8a8: the reference's default W8A8 text linears (int8 weights and activations;
    the LM head stays bf16), reported beside the bf16 figures, never as them."""
    import torch
    import strix_halo_maxx_amd.md2text as mt
    import strix_halo_maxx_amd.synth as S
    dev = torch.device("cuda:0")
    w = S.text_weights(0)
    # yes / no ids: 4 + 4 fixed ids (no tokenizer here); nq = 1 question of up to L = 32 ids (the reference's
    # FastMD2 defaults, md2fast.py:69)
    dec = mt.TextDecoder(w, device=dev, ctx=1024, w8a8=w8a8, yes_ids=(11, 222, 3333, 44444),
                         no_ids=(55, 666, 7777, 50000))
    del w
    img = S.activations(3, (729, 2048), "img").to(dev)
    prompt = S.prompt_ids(4, 64)
    for _ in range(2):
        dec.generate(img, prompt, 8)
    torch.cuda.synchronize()

    def time_prefill(n):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            dec.prefill(img, prompt)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[n // 2]
    t_pre_eager = time_prefill(3)  # eager launches (host-bound part included)
    dec.capture_prefill(img.shape[0], prompt.shape[0])  # prefix + prompt + LM head as one HIP graph
    t_pre = time_prefill(10)

    def time_decode():
        dec.prefill(img, prompt)
        dec.start_decode()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps_tokens - 1):
            dec.replay_step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / (steps_tokens - 1)
    t_dec = time_decode()
    path = ("one launch per step (mx_decode_step_mk" + ("_i8)" if w8a8 else ")")) if dec.use_mk else "per-layer kernels"
    if dec.mk_error():
        raise RuntimeError(f"one-launch decode step reported error {dec.mk_error()}")
    t_layers = None
    if dec.use_mk:  # the per-layer kernel sequence beside it, on the same decoder
        dec.use_mk = False
        dec.graph = None
        for _ in range(2):
            dec.generate(img, prompt, 8)
        t_layers = time_decode()
        dec.use_mk = True
    # the reference's yes/no query (FastMD2.query, md2fast.py:208-212): a 32-id question over the 730-token prefix,
    # yes / no rows of the LM head, one HIP graph
    dec.encode(img)
    dec.set_questions([prompt[:32].tolist()])
    dec.capture_query()
    for _ in range(3):
        dec.query()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        dec.query()
    torch.cuda.synchronize()
    t_q = (time.perf_counter() - t0) / 20
    c = S.TXT
    D, F, L, V = c["dim"], c["ff"], c["layers"], c["vocab"]
    lin = L * (3 * D * D + D * D + 2 * D * F)  # text Linear weights: bf16, or int8 + fp32 per-row scales (W8A8)
    wbytes = (lin + 4 * L * (3 * D + D + F + D) if w8a8 else 2 * lin) + 2 * V * D
    ctx_mid = dec.pos_base + steps_tokens // 2
    kvbytes = 2 * 2 * L * ctx_mid * D
    bpt = wbytes + kvbytes
    traffic = {}
    mt_ = measured_decode_traffic() if dec.use_mk and not w8a8 else None
    if mt_:  # counted HBM bytes of one step over its algorithmic bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE)
        traffic = {"traffic_per_step": mt_[0], "traffic_ratio": round(mt_[0] / mt_[1], 4),
                   "traffic_source": os.path.relpath(DECODE_TRAFFIC_FILE, os.path.dirname(DECODE_TRAFFIC_FILE) + "/..")}
    fl_pre = 2 * L * (D * 3 * D + D * D + 2 * D * F) * (730 + 64) + 2 * 2 * L * D * (730 * 730 + 64 * (730 + 64))
    return {"prefill_ms": round(t_pre * 1e3, 3), "prefill_ms_eager": round(t_pre_eager * 1e3, 3),
            "prefill_mfma_frac": round(fl_pre / t_pre / PEAK_BF16, 4),
            "query_ms": round(t_q * 1e3, 3), "decode_tok_s": round(1.0 / t_dec, 1),
            "decode_ms_per_token": round(t_dec * 1e3, 4), "decode_path": path,
            "decode_tok_s_layer_kernels": round(1.0 / t_layers, 1) if t_layers else None,
            "decode_roofline": {"bound": "hbm", "achieved": round(bpt / t_dec / 1e9, 1), "peak": PEAK_HBM / 1e9,
                                "unit": "GB/s", "frac": round(bpt / t_dec / PEAK_HBM, 4),
                                "bytes_per_token": bpt, **traffic},
            "workload": "moondream2 text decoder, 24 layers, prefill 730 + 64 tokens (one HIP graph; eager beside it), "
                        f"greedy {steps_tokens} tokens, batch 1, one HIP graph per decode step; query_ms: one 32-id "
                        "yes/no query over the 730-token prefix (graph)"
                        + (", W8A8 text Linears (int8 weights / activations, bf16 LM head)" if w8a8 else "")}


def frame_bench(reps=20):
    """The whole moondream2 yes/no frame (FastMD2, md2fast.py:147-160, 201-212): vision tower at batch 1 +
    projection MLP + 730-token prefix prefill (one HIP graph), then one 32-id question over it with the yes / no rows
    of the LM head (a second graph). ms per frame = both replays; the reference publishes 88.7 ms for the same frame
    on its own GPU (moondream/gpu/README.md:11-13)."""
    import torch
    import strix_halo_maxx_amd.md2frame as mf
    import strix_halo_maxx_amd.synth as S
    dev = torch.device("cuda:0")
    f = mf.FastMD2(S.vision_weights(0, proj=True), S.text_weights(0), device=dev, nq=1, L=32,
                   yes_ids=(11, 222, 3333, 44444), no_ids=(55, 666, 7777, 50000))
    img = S.images_u8(1, 1)[0].to(dev)
    f.set_questions([S.prompt_ids(4, 32).tolist()])
    f.img.copy_(img)
    f.capture()
    for _ in range(3):
        f.frame(img)
    torch.cuda.synchronize()
    t = {}
    for name, fn in (("encode", lambda: f.encode(img)), ("query", f.query), ("frame", lambda: f.frame(img))):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        t[name] = (time.perf_counter() - t0) / reps * 1e3
    return {"frame_ms": round(t["frame"], 3), "encode_ms": round(t["encode"], 3), "query_ms": round(t["query"], 3),
            "workload": "moondream2 yes/no frame: vision tower (27 blocks, batch 1) + projection MLP + 730-token "
                        "prefix prefill (24 text layers), then one 32-id question + yes/no head; two HIP graphs"}


def trecvit_bench(frames=64, clip=16):
    """Config 3: TRecViT, 12 blocks, 1024 patch + 256 query tokens, streamed for `frames` frames (one HIP graph per
    frame), plus the clip-parallel form (`clip` frames per pass through every block)."""
    import torch
    import strix_halo_maxx_amd.synth as S
    import strix_halo_maxx_amd.trecvit as tv
    dev = torch.device("cuda:0")
    m = tv.TRecViT(S.trecvit_weights(0), device=dev)
    fr = S.frames_u8(1, frames).to(dev)
    q = S.query_points(5, 256)
    qf = (q[:, 1:] / 256.0).to(torch.bfloat16).to(dev)
    m.reset()
    for t in range(4):
        m.step(fr[t], qf)  # eager warm-up (GEMM tile tuning)
    m.reset()
    m.capture()
    for t in range(4):
        m.step(fr[t], qf, use_graph=True)
    m.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(frames):
        m.step(fr[t], qf, use_graph=True)
    torch.cuda.synchronize()
    ms_stream = (time.perf_counter() - t0) / frames * 1e3
    if m.rln_error():  # a timed-out row-block wait of the fused residual-LayerNorm GEMM leaves undefined results
        raise RuntimeError(f"fused residual-LayerNorm GEMM reported error {m.rln_error()}")
    m.graphs.clear()
    m.reset()
    m.clip_state(clip)
    m.forward_clip(fr[:clip], qf)
    m.reset()
    m.clip_state(clip)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for c0 in range(0, frames, clip):
        m.forward_clip(fr[c0:c0 + clip], qf)
    torch.cuda.synchronize()
    ms_clip = (time.perf_counter() - t0) / frames * 1e3
    scan = scan_roofline(m, clip)
    c = S.TRV
    T, D = 1280, c["dim"]
    gemm = 2 * T * (D * 2 * D + D * D + D * 2 * c["ff_gated"] + c["ff_gated"] * D + D * 3 * D + D * D + 2 * D * c["ff_vit"])
    attn = 4 * T * T * D
    gates = 2 * 2 * T * D * 64
    fl = c["layers"] * (gemm + attn + gates)
    return {"stream_ms_per_frame": round(ms_stream, 3), "clip_ms_per_frame": round(ms_clip, 3), "clip_frames": clip,
            "frames": frames, "gflop_per_frame": round(fl / 1e9, 1),
            "stream_mfma_frac": round(fl / (ms_stream / 1e3) / PEAK_BF16, 4),
            "clip_mfma_frac": round(fl / (ms_clip / 1e3) / PEAK_BF16, 4), "scan_roofline": scan,
            "workload": "TAPNext-style TRecViT, 12 blocks, hidden 768, 1024 patch + 256 query tokens, 64 frames"}


def scan_roofline(m, F, launches=24):
    """HBM roofline of the RG-LRU time scan (mx_rglru_scan) at the clip shape: F frames x 1280 tokens x 768
    channels. Algorithmic bytes per launch: A, B (fp32) and yg (bf16) read and z (bf16) written per (frame, token,
    channel), the fp32 state read and written once: 12 F T C + 8 T C. Timed with HIP events on the launching stream
    over `launches` launches, each on its own buffers (cold: 24 x 160 MB is far past the 256 MB MALL)."""
    import torch
    from strix_halo_maxx_amd import _lib
    dev, T, C = m.dev, m.T, m.D
    g = torch.Generator(device=dev).manual_seed(3)
    bufs = []
    for _ in range(launches):
        A = torch.rand(F, T, C, device=dev, generator=g)
        B = torch.randn(F, T, C, device=dev, generator=g)
        yg = torch.randn(F, T, 2 * C, device=dev, generator=g).to(torch.bfloat16)
        bufs.append((A, B, torch.zeros(T, C, device=dev), yg, torch.empty(F, T, C, device=dev, dtype=torch.bfloat16)))
    run = lambda b: _lib.call("mx_rglru_scan", _lib.stream(), b[0].data_ptr(), b[1].data_ptr(), b[2].data_ptr(), F,
                              T, C, b[3].data_ptr(), 2 * C, T * 2 * C, b[4].data_ptr(), C, T * C)
    for b in bufs[:2]:
        run(b)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for b in bufs:
        run(b)
    e1.record(st)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    nbytes = 12 * F * T * C + 8 * T * C
    del bufs
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "rglru_chain_kernel", "achieved": round(nbytes / us / 1e3, 1),
            "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(nbytes / us / 1e3 / (PEAK_HBM / 1e9), 4),
            "avg_launch_us": round(us, 2), "bytes_per_launch": nbytes}


def large_batch_ops(vt, imgs, reps=5):
    """Per-op launch time of one tower block at a large batch (the throughput-bound config: its GEMMs run the
    large-M tiles, not the batch-1 split-K path): qkv, attention, proj (+ residual), LN, fc1 (+ GELU), fc2
    (+ residual), each on block 0's real operands, `reps` launches between HIP events on the launching stream.
    Returns {op: {"us", "tflops", "mfma_frac"}} (LN: GB/s instead)."""
    import torch
    ops_ = large_batch_block_ops(vt, imgs)
    M, D = imgs.shape[0] * vt.T, vt.D
    st = torch.cuda.current_stream()
    res = {}
    for name, (fl, _, fn) in ops_.items():
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            fn()
        e1.record(st)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        if fl:
            res[name] = {"us": round(us, 1), "tflops": round(fl / us / 1e6, 1), "mfma_frac": round(fl / us / 1e6 / (PEAK_BF16 / 1e12), 4)}
        else:
            res[name] = {"us": round(us, 1), "gb_s": round(4 * M * D / us / 1e3, 1)}
    gemm_fl = sum(ops_[k][0] for k in ("qkv", "proj", "fc1", "fc2"))
    gemm_us = sum(res[k]["us"] for k in ("qkv", "proj", "fc1", "fc2"))
    res["gemms"] = {"tflops": round(gemm_fl / gemm_us / 1e6, 1), "mfma_frac": round(gemm_fl / gemm_us / 1e6 / (PEAK_BF16 / 1e12), 4)}
    return res


def large_batch_block_ops(vt, imgs):
    """Block 0's ops at a large batch on its real operands: {op: (flops, algorithmic HBM bytes, fn)}, fn relaunching
    the op into fixed outputs (every operand once: bf16 activations and weights)."""
    import torch
    import strix_halo_maxx_amd.ops as ops
    B = imgs.shape[0]
    T, D, H, hd = vt.T, vt.D, vt.H, vt.hd
    M = B * T
    b = vt.blocks[0]
    x = vt.embed(imgs)
    h = ops.layernorm(x, *b["ln1"], eps=vt.eps)
    qkv = b["qkv"](h)
    q5 = qkv.view(B, T, 3, H, hd)
    q, k, v = (q5[:, :, j].transpose(1, 2) for j in range(3))
    a = vt.attn(q, k, v).view(M, D)
    x1 = b["proj"](a, res=x)
    h2 = ops.layernorm(x1, *b["ln2"], eps=vt.eps)
    f = b["fc1"](h2, gelu=True)
    F = f.shape[1]
    y = torch.empty_like(x)
    return {"qkv": (2 * M * D * 3 * D, 2 * (M * D + 3 * D * D + 3 * M * D), lambda: b["qkv"](h, out=qkv)),
            "attn": (4 * B * H * T * T * hd, 2 * 4 * M * D, lambda: ops.sdpa(q, k, v, out=a.view(B, T, D))),
            "proj": (2 * M * D * D, 2 * (3 * M * D + D * D), lambda: b["proj"](a, res=x, out=y)),
            "ln": (0, 2 * 2 * M * D, lambda: ops.layernorm(x1, *b["ln2"], eps=vt.eps, out=h2)),
            "fc1": (2 * M * D * F, 2 * (M * D + F * D + M * F), lambda: b["fc1"](h2, gelu=True, out=f)),
            "fc2": (2 * M * F * D, 2 * (M * F + D * F + 2 * M * D), lambda: b["fc2"](f, res=x1, out=y))}


PROBES = ("tower_b256", "trecvit", "scan", "decode_w8a8", "prefill")


def _probe_classes(workload):
    """Launch classes of a profiling probe: (title, [(label, fn, algorithmic HBM bytes per call or None, flops per
    call)]), built on the device with every warm-up (tile tuning, first-touch) done. fn() launches one call of the
    class eagerly (no graph)."""
    import torch
    import strix_halo_maxx_amd.synth as S
    dev = torch.device("cuda:0")
    if workload == "tower_b256":
        import strix_halo_maxx_amd.md2 as md2
        vt = md2.VisionTower(S.vision_weights(0), device=dev)
        imgs = S.images_u8(2, 256).to(dev)
        vt(imgs)
        ops_ = large_batch_block_ops(vt, imgs)
        for _, _, fn in ops_.values():
            fn()
        return ("moondream2 vision tower at batch 256 (186,624 tokens), block 0's ops on its own operands",
                [(k, fn, algo, fl) for k, (fl, algo, fn) in ops_.items()])
    if workload == "trecvit":
        import strix_halo_maxx_amd.trecvit as tv
        m = tv.TRecViT(S.trecvit_weights(0), device=dev)
        fr = S.frames_u8(1, 4).to(dev)
        qf = (S.query_points(5, 256)[:, 1:] / 256.0).to(torch.bfloat16).to(dev)
        m.reset()
        for t in range(3):
            m.step(fr[t], qf)
        return ("TRecViT streamed frame (12 blocks, 1024 patch + 256 query tokens, hidden 768) with the tracking "
                "heads, eager launches", [("frame", lambda: m.step(fr[3], qf), None, None)])
    if workload == "scan":
        T, C, F = 1280, 768, 16
        g = torch.Generator(device=dev).manual_seed(3)
        bufs = [(torch.rand(F, T, C, device=dev, generator=g), torch.randn(F, T, C, device=dev, generator=g),
                 torch.zeros(T, C, device=dev),
                 torch.randn(F, T, 2 * C, device=dev, generator=g).to(torch.bfloat16),
                 torch.empty(F, T, C, device=dev, dtype=torch.bfloat16)) for _ in range(4)]
        it = iter(range(1 << 30))
        from strix_halo_maxx_amd import _lib

        def run():
            b = bufs[next(it) % len(bufs)]
            _lib.call("mx_rglru_scan", _lib.stream(), b[0].data_ptr(), b[1].data_ptr(), b[2].data_ptr(), F, T, C,
                      b[3].data_ptr(), 2 * C, T * 2 * C, b[4].data_ptr(), C, T * C)
        run()
        return (f"RG-LRU clip scan (mx_rglru_scan, {F} frames x {T} tokens x {C} channels), each call on its own "
                "buffers", [("scan", run, 12 * F * T * C + 8 * T * C, None)])
    if workload == "decode_w8a8":
        import strix_halo_maxx_amd.md2text as mt
        dec = mt.TextDecoder(S.text_weights(0), device=dev, ctx=1024, w8a8=True)
        if not dec.use_mk:
            raise RuntimeError("the one-launch decode step is not in use on this device")
        img = S.activations(3, (729, 2048), "img").to(dev)
        prompt = S.prompt_ids(4, 64)
        dec.generate(img, prompt, 4)
        dec.prefill(img, prompt)
        dec.start_decode()
        for _ in range(2):
            dec.decode_step()
        c = S.TXT
        D, F_, L, V = c["dim"], c["ff"], c["layers"], c["vocab"]
        lin = L * (3 * D * D + D * D + 2 * D * F_)
        algo = lin + 4 * L * (3 * D + D + F_ + D) + 2 * V * D + 2 * 2 * L * (dec.pos_base + 3) * D
        return ("moondream2 W8A8 one-launch decode step (mx_decode_step_mk_i8), 24 layers, from position "
                f"{dec.pos_base + 2}", [("step", dec.decode_step, algo, None)])
    if workload == "prefill":
        import strix_halo_maxx_amd.md2text as mt
        dec = mt.TextDecoder(S.text_weights(0), device=dev, ctx=1024)
        img = S.activations(3, (729, 2048), "img").to(dev)
        prompt = S.prompt_ids(4, 64)
        for _ in range(2):
            dec.prefill(img, prompt)
        c = S.TXT
        D, F_, L = c["dim"], c["ff"], c["layers"]
        n, P = 729 + 1 + 64, 730
        fl = 2 * L * (3 * D * D + D * D + 2 * D * F_) * n + 4 * L * D * (P * P + (n - P) * n)
        return ("moondream2 text prefill, 24 layers, 730 prefix + 64 prompt rows in one pass, eager launches",
                [("prefill", lambda: dec.prefill(img, prompt), None, fl)])
    raise ValueError(f"unknown probe {workload}; one of {PROBES}")


def probe(workload, reps=3):
    """Eager launches for rocprofv3 --pmc passes over one workload: after the warm-ups, for class i a marker fill of
    10000 + i int16 values (a fill kernel no workload runs: FillFunctor<short>) then `reps` calls of the class; then
    a marker fill of 99999 int16 values and the calibration: `reps` device copies of 256 MiB (known traffic: 256 MiB
    read + 256 MiB written each)."""
    import torch
    title, classes = _probe_classes(workload)
    torch.cuda.synchronize()
    for i, (label, fn, _, _) in enumerate(classes):
        torch.full((10000 + i,), 1, dtype=torch.int16, device="cuda:0")
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
    torch.full((99999,), 1, dtype=torch.int16, device="cuda:0")
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] probe {workload} done: {title}", flush=True)


def _pmc_dispatches(path):
    """{counter: [(kernel, grid threads, value)] in dispatch order} from a rocprofv3 counter_collection CSV (values
    of one dispatch summed over their dimension rows; MfmaUtil, a percentage, averaged)."""
    import csv
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            c = r["Counter_Name"]
            d = int(r["Dispatch_Id"])
            k = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "")
            k = k[:k.rfind(">") + 1] if ">" in k else k.split("(")[0]
            e = per.setdefault(c, {}).setdefault(d, [k, int(r.get("Grid_Size", 0) or 0), 0.0, 0])
            e[2] += float(r["Counter_Value"])
            e[3] += 1
    out = {}
    for c, m in per.items():
        out[c] = [(k, g, v / n if c == "MfmaUtil" else v) for _, (k, g, v, n) in sorted(m.items())]
    return out


def summarize_probe(workload, paths, reps=3):
    """Markdown summary of rocprofv3 --pmc passes (one CSV each) over `bench.py --probe WORKLOAD`: per class, per
    (kernel, grid): dispatches per call, HBM traffic per dispatch from FETCH_SIZE / WRITE_SIZE (scaled by what the
    counters read for the 256 MiB calibration copies), and whichever of MfmaUtil, the waiting / issue fractions of
    wave time, LDS bank conflicts and the L2 hit rate the CSVs hold."""
    title, classes = _probe_classes(workload)
    vals = {}
    for p in paths:
        vals.update(_pmc_dispatches(p))
    segs = {}
    for c, seq in vals.items():
        fills = [i for i, (k, _, _) in enumerate(seq) if "FillFunctor<short>" in k]
        marks = fills[-(len(classes) + 1):]
        if len(marks) != len(classes) + 1:
            raise RuntimeError(f"{c}: {len(fills)} marker fills for {len(classes)} classes")
        parts = [seq[marks[i] + 1:marks[i + 1]] for i in range(len(classes))]
        segs[c] = (parts, [v for k, _, v in seq[marks[-1] + 1:] if "copyBuffer" in k][:reps])
    cal = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        if c in segs:
            cp = segs[c][1]
            if len(cp) < reps:
                raise RuntimeError(f"{c}: {len(cp)} calibration copies")
            cal[c] = (256 << 20) / (sum(cp) / reps * 1024)
    rows, blob = [], {"workload": workload, "title": title, "calibration": {k: round(v, 4) for k, v in cal.items()},
                      "kernels": []}
    any_c = next(iter(segs))
    for j, (label, _, algo, fl) in enumerate(classes):
        order = []
        groups = {}
        for idx, (k, g, _) in enumerate(segs[any_c][0][j]):
            key = (k, g)
            if key not in groups:
                order.append(key)
                groups[key] = []
            groups[key].append(idx)
        for key in order:
            idxs = groups[key]
            stat = lambda c: sum(segs[c][0][j][i][2] for i in idxs) / len(idxs) if c in segs else None
            e = {"class": label, "kernel": key[0], "grid_threads": key[1], "dispatches_per_call": len(idxs) / reps}
            if cal:
                rd, wr = stat("FETCH_SIZE") * 1024 * cal["FETCH_SIZE"], stat("WRITE_SIZE") * 1024 * cal["WRITE_SIZE"]
                e.update(read_bytes=int(rd), write_bytes=int(wr))
            for c in ("MfmaUtil", "SQ_WAIT_ANY", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_VALU",
                      "SQ_ACTIVE_INST_LDS", "SQ_LDS_BANK_CONFLICT", "TCC_HIT_sum", "TCC_MISS_sum"):
                if c in segs:
                    e[c] = stat(c)
            if algo and len(order) == 1:
                e["algorithmic_bytes"] = algo
            if fl and len(order) == 1:
                e["flops"] = fl
            blob["kernels"].append(e)
    cols = [("dispatches / call", lambda e: f"{e['dispatches_per_call']:g}")]
    if cal:
        cols += [("read MB", lambda e: f"{e['read_bytes'] / 1e6:,.2f}"), ("written MB", lambda e: f"{e['write_bytes'] / 1e6:,.2f}"),
                 ("algorithmic MB", lambda e: f"{e['algorithmic_bytes'] / 1e6:,.2f}" if "algorithmic_bytes" in e else "")
                 , ("traffic / algorithmic", lambda e: f"{(e['read_bytes'] + e['write_bytes']) / e['algorithmic_bytes']:.2f}"
                    if "algorithmic_bytes" in e else "")]
    have = set(blob["kernels"][0]) if blob["kernels"] else set()
    if "MfmaUtil" in have:
        cols.append(("MfmaUtil %", lambda e: f"{e['MfmaUtil']:.1f}"))
    if "SQ_WAVE_CYCLES" in have:
        for c, lab in (("SQ_WAIT_ANY", "waiting / wave time"), ("SQ_WAIT_INST_ANY", "issue-stalled / wave time"),
                       ("SQ_ACTIVE_INST_VALU", "VALU + MFMA issue / wave time"),
                       ("SQ_ACTIVE_INST_LDS", "LDS issue / wave time")):
            if c in have:
                cols.append((lab, lambda e, c=c: f"{e[c] / e['SQ_WAVE_CYCLES']:.2f}" if e["SQ_WAVE_CYCLES"] else ""))
    if "SQ_LDS_BANK_CONFLICT" in have:
        cols.append(("LDS bank-conflict cycles", lambda e: f"{e['SQ_LDS_BANK_CONFLICT']:,.0f}"))
    if "TCC_HIT_sum" in have and "TCC_MISS_sum" in have:
        cols.append(("L2 hit rate", lambda e: f"{e['TCC_HIT_sum'] / max(1.0, e['TCC_HIT_sum'] + e['TCC_MISS_sum']):.2f}"))
    lines = ["| class | kernel | grid threads | " + " | ".join(c for c, _ in cols) + " |",
             "|" + "---|" * (len(cols) + 3)]
    for e in blob["kernels"]:
        lines.append(f"| {e['class']} | `{e['kernel'][:70]}` | {e['grid_threads']:,} | " +
                     " | ".join(fn(e) for _, fn in cols) + " |")
    head = f"Workload: {title}.\n\n"
    if cal:
        head += (f"Calibration: a 256 MiB device copy reads {256 * 1024 / cal['FETCH_SIZE']:,.1f} KiB of FETCH_SIZE and "
                 f"{256 * 1024 / cal['WRITE_SIZE']:,.1f} KiB of WRITE_SIZE; bytes = FETCH_SIZE x 1024 x "
                 f"{cal['FETCH_SIZE']:.4f} + WRITE_SIZE x 1024 x {cal['WRITE_SIZE']:.4f}.\n\n")
    return head + "\n".join(lines) + "\n\n```json\n" + json.dumps(blob, indent=1, default=float) + "\n```\n"


def tower_time(vt, img, steps, warmup):
    import torch
    for _ in range(warmup):
        vt(img)
    g, out = vt.capture(img)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline tower only (no batch 13 / 256, decoder, TRecViT)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only the eager launches that rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs count (see traffic_probe)")
    ap.add_argument("--traffic-probe-decode", action="store_true",
                    help="only the eager one-launch decode steps the --pmc passes count (see traffic_probe_decode)")
    ap.add_argument("--summarize-traffic-decode", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic summary of two --pmc passes over --traffic-probe-decode")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic summary of two --pmc passes over --traffic-probe (see summarize_traffic)")
    ap.add_argument("--summarize-trace", metavar="TRACE_CSV", help="print a rocprofv3 kernel trace grouped by kernel")
    ap.add_argument("--summarize-counters", nargs="+", metavar="PMC_CSV",
                    help="print per-op MFMA / wait / LDS / L2 counters of --pmc passes over --traffic-probe")
    ap.add_argument("--probe", choices=PROBES, help="only the eager launches of one workload that rocprofv3 --pmc "
                    "passes count (see probe)")
    ap.add_argument("--summarize-probe", nargs="+", metavar=("WORKLOAD", "PMC_CSV"),
                    help="print the per-kernel summary of --pmc passes (one CSV each) over --probe WORKLOAD")
    a = ap.parse_args()
    if a.summarize_probe:
        import torch
        with torch.inference_mode():
            print(summarize_probe(a.summarize_probe[0], a.summarize_probe[1:]))
        return
    if a.probe:
        import torch
        with torch.inference_mode():
            probe(a.probe)
        return
    if a.summarize_counters:
        print(summarize_counters(a.summarize_counters))
        return
    if a.summarize_trace:
        print(summarize_trace(a.summarize_trace))
        return
    if a.summarize_traffic:
        print(summarize_traffic(*a.summarize_traffic))
        return
    if a.summarize_traffic_decode:
        print(summarize_traffic_decode(*a.summarize_traffic_decode))
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (every workload here fits one GPU's "
              "288 GB; the sharding plan is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import strix_halo_maxx_amd.md2 as md2
    import strix_halo_maxx_amd.synth as S

    if a.traffic_probe_decode:
        with torch.inference_mode():
            traffic_probe_decode()
        return
    dev = torch.device("cuda:0")
    w = S.vision_weights(0)
    vt = md2.VisionTower(w, device=dev)
    img = S.images_u8(1, 1).to(dev)
    if a.traffic_probe:
        with torch.inference_mode():
            traffic_probe(vt, img)
        return
    print(f"[bench] tower batch 1: warmup {a.warmup}, steps {a.steps}", file=sys.stderr, flush=True)
    with torch.inference_mode():
        s = tower_time(vt, img, a.steps, a.warmup)
        agg = op_timing(vt, img)
    if vt.rln_error():  # a timed-out row-block wait of the fused residual-LayerNorm GEMM leaves undefined results
        raise RuntimeError(f"fused residual-LayerNorm GEMM reported error {vt.rln_error()}")
    ms = s * 1e3
    label, (tot_ms, n, fl, sym) = max(agg.items(), key=lambda kv: kv[1][0])
    avg_s = tot_ms / n / 1e3
    achieved = fl / avg_s
    traffic, tsrc = measured_traffic(label, sym)
    roof = {"bound": "mfma", "kernel": sym, "op": label, "achieved": round(achieved / 1e12, 1),
            "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4), "traffic": traffic,
            "traffic_source": tsrc,
            "avg_launch_us": round(avg_s * 1e6, 2), "launches_timed": n, "flops_per_launch": fl,
            "per_op_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in agg.items()},
            "per_op_kernel": {k: v[3] for k, v in agg.items()}}
    tower_flops = vision_flops_per_frame()
    out = {"metric": "ms/frame moondream2 vision tower bs=1; decode tok/s; % MFMA / HBM roofline", "value": round(ms, 4), "unit": "ms/frame", "n_gpus": 1,
           "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded u8 pixels, N(0,0.02) weights)",
           "config": {"workload": "moondream2 SigLIP vision tower, 27 blocks + post-LN, 729 tokens, batch 1, HIP graph",
                      "batch": 1, "tokens": 729, "layers": 27},
           "tower_tflops": round(tower_flops / s / 1e12, 1), "tower_mfma_frac": round(tower_flops / s / PEAK_BF16, 4),
           "roofline": roof}
    if not a.no_extra:
        print("[bench] tower batch 13 / 256", file=sys.stderr, flush=True)
        with torch.inference_mode():
            for B in (13, 256):
                imgs = S.images_u8(2, B).to(dev)
                # ~0.3 s of timed replays each: 25 batches of 13, 5 of 256 at the default 50 steps
                sb = tower_time(vt, imgs, max(5, a.steps // 2) if B == 13 else max(3, a.steps // 10), 2)
                out.setdefault("extra", {})[f"tower_b{B}"] = {"ms_per_batch": round(sb * 1e3, 3),
                                                              "images_per_s": round(B / sb, 1),
                                                              "mfma_frac": round(B * tower_flops / sb / PEAK_BF16, 4)}
                if B == 256:
                    vt.graphs.clear()
                    out["extra"]["tower_b256"]["per_op_block0"] = large_batch_ops(vt, imgs)
                del imgs
                vt.graphs.clear()
                torch.cuda.empty_cache()
        if vt.rln_error():
            raise RuntimeError(f"fused residual-LayerNorm GEMM reported error {vt.rln_error()}")
    del vt
    torch.cuda.empty_cache()
    if not a.no_extra:
        print("[bench] one vision block", file=sys.stderr, flush=True)
        with torch.inference_mode():
            out.setdefault("extra", {})["vision_block"] = block_bench(cpu=not a.no_cpu)
        torch.cuda.empty_cache()
        print("[bench] decoder", file=sys.stderr, flush=True)
        with torch.inference_mode():
            out.setdefault("extra", {})["decoder"] = decode_bench()
        torch.cuda.empty_cache()
        print("[bench] decoder w8a8", file=sys.stderr, flush=True)
        with torch.inference_mode():
            out["extra"]["decoder_w8a8"] = decode_bench(w8a8=True)
        torch.cuda.empty_cache()
        print("[bench] moondream2 yes/no frame", file=sys.stderr, flush=True)
        with torch.inference_mode():
            out["extra"]["md2_frame"] = frame_bench()
        torch.cuda.empty_cache()
        print("[bench] trecvit", file=sys.stderr, flush=True)
        with torch.inference_mode():
            out["extra"]["trecvit"] = trecvit_bench()
    if not a.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline()
        if not a.no_extra:
            print("[bench] cpu baseline: decoder, trecvit", file=sys.stderr, flush=True)
            out["extra"]["decoder"]["cpu_baseline"] = cpu_baseline_decoder()
            out["extra"]["trecvit"]["cpu_baseline"] = cpu_baseline_trecvit()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
