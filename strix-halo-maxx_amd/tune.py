"""Build the fixed GEMM tile table for MI355X (gemm_table_gfx950.json next to this file).

    python -m strix_halo_maxx_amd.tune [--reps 5]

The batch-1 vision tower is tuned in context: for every GEMM op class (qkv, fc1: fused epilogues; proj, fc2: split-K
partials reduced by the residual-LayerNorm kernel), each candidate (tile config, split count) is timed on the 27
launches of that op across the tower's blocks, each on its own block's weights, replayed from a HIP graph. That is the
cost the op has inside the tower, where a block's weights arrive from HBM rather than from a cache warmed by the
previous launch; the split-K candidates are timed together with the reduction kernel that reads their partials. The
other shapes (tower batch 13 / 256, text-decoder prefill and yes/no query, TRecViT stream and clip passes) come from the generic
per-shape autotuner (ops.tune_gemm, ops._partial_cfg) run on their own forwards. The result is written as JSON;
ops.MxLin then uses it before autotuning (the reference's pick_cfg FIXED table, moondream/gpu/hgemm.py:47-76).
"""
import argparse
import json
import os
import sys

import torch

from . import ops, _lib
from . import md2, md2text, trecvit
from . import synth as S


def _time_graph(fn, reps):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    e1.synchronize()
    del g
    return e0.elapsed_time(e1) / reps


def _refine(cands, reps, log, name, rounds=3, top=4):
    """Re-time the `top` fastest (time, pick, fn) candidates `rounds` times, interleaved, with 4x the reps, and return
    the pick with the lowest median: first-sweep margins of ~1 % between tile configs are within run-to-run noise."""
    cands = sorted(cands, key=lambda c: c[0])[:top]
    ts = {c[1]: [] for c in cands}
    for _ in range(rounds):
        for _, pick, fn in cands:
            ts[pick].append(_time_graph(fn, 4 * reps))
    med = {k: sorted(v)[len(v) // 2] for k, v in ts.items()}
    best = min(med, key=med.get)
    log(f"tower {name} refined: " + ", ".join(f"{k}: {v * 1e3:.1f} us" for k, v in med.items()) + f" -> {best}")
    return best


def tune_tower_b1(reps, log):
    """In-context table entries for the batch-1 tower: {(M, N, Kw): (cfg, splits)} fused and partial."""
    dev = torch.device("cuda:0")
    vt = md2.VisionTower(S.vision_weights(0), device=dev)
    img = S.images_u8(1, 1).to(dev)
    lib = _lib.load()
    ncfg = lib.mx_gemm_ncfg()
    B, T, D, H, hd = 1, vt.T, vt.D, vt.H, vt.hd
    M = B * T
    blocks = vt.blocks
    with torch.inference_mode():
        vt(img)  # generic tuning of every shape, so the eager pass below has configs to run with
        saved = []
        x = vt.embed(img)
        h = ops.layernorm(x, *blocks[0]["ln1"], eps=vt.eps)
        for i, b in enumerate(blocks):
            a = vt._attn(b, h, B)
            pp = b["proj"].partial(a)
            x1, h2 = ops.residual_layernorm(pp, b["proj"].b, x, b["ln2"], eps=vt.eps)
            f = b["fc1"](h2, gelu=True)
            pf = b["fc2"].partial(f)
            nxt = blocks[i + 1]["ln1"] if i + 1 < len(blocks) else vt.post_ln
            x2, hn = ops.residual_layernorm(pf, b["fc2"].b, x1, nxt, eps=vt.eps)
            saved.append((x, h, a, x1, h2, f, nxt))
            x, h = x2, hn
        fused, part = {}, {}
        # ---- fused-epilogue ops
        for name, act, inp in (("qkv", 0, 1), ("fc1", 1, 4)):
            lin0 = blocks[0][name]
            out = torch.empty(M, lin0.N, device=dev, dtype=torch.bfloat16)
            cands = []
            for cfg in range(ncfg):
                def run(cfg=cfg, name=name, act=act, inp=inp):
                    for i, b in enumerate(blocks):
                        b[name].cfgs[M] = (cfg, 1)
                        b[name](saved[i][inp], gelu=bool(act), out=out)
                try:
                    t = _time_graph(run, reps)
                except _lib.MxError:
                    continue
                log(f"tower {name} cfg {cfg}: {t * 1e3 / len(blocks):.2f} us/launch")
                cands.append((t, (cfg, 1), run))
            best = _refine(cands, reps, log, name)
            for b in blocks:
                b[name].cfgs.pop(M, None)
            fused[(M, lin0.N, lin0.Kw)] = best
            log(f"tower {name}: pick {best}")
        # ---- split-K ops, timed with the residual-LayerNorm that reduces them
        for name, inp, resi, ln in (("proj", 2, 0, "ln2"), ("fc2", 5, 3, None)):
            lin0 = blocks[0][name]
            key = (M, lin0.N, lin0.Kw)
            nk = lin0.Kw // 64
            xo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)
            yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)
            cands = []
            for cfg in range(ncfg):
                for sp in (1, 2, 3, 4):
                    if sp > 1 and (nk // sp < 2 or (sp - 1) * (-(-nk // sp)) >= nk):
                        continue
                    P = torch.empty(sp, M, lin0.N, device=dev, dtype=torch.float32)
                    if ops._partial(lin0, cfg, sp, ops._rows(saved[0][inp], lin0.K), P, M) != 0:
                        continue  # no partial-sum mode for this config

                    def run(cfg=cfg, sp=sp, P=P, name=name, inp=inp, resi=resi, ln=ln, key=key):
                        ops._TUNED_P[key] = (cfg, sp)
                        for i, b in enumerate(blocks):
                            lnp = b[ln] if ln else saved[i][6]
                            ops.residual_layernorm(b[name].partial(saved[i][inp], out=P), b[name].b, saved[i][resi],
                                                   lnp, eps=vt.eps, x_out=xo, y_out=yo)
                    t = _time_graph(run, reps)
                    log(f"tower {name} cfg {cfg} x{sp}: {t * 1e3 / len(blocks):.2f} us/launch (with the reduction)")
                    cands.append((t, (cfg, sp), run))
            best = _refine(cands, reps, log, name)
            ops._TUNED_P.pop(key, None)
            part[key] = best
            log(f"tower {name}: pick {best}")
    del vt
    torch.cuda.empty_cache()
    return fused, part


def tune_generic(log):
    """Autotuner picks for the other workloads' shapes (their own forwards, tuned on first use)."""
    dev = torch.device("cuda:0")
    before, before_p = set(ops._TUNED), set(ops._TUNED_P)
    with torch.inference_mode():
        vt = md2.VisionTower(S.vision_weights(0), device=dev)
        for B in (13, 256):
            vt(S.images_u8(2, B).to(dev))
            torch.cuda.synchronize()
            log(f"tower batch {B} tuned")
        del vt
        torch.cuda.empty_cache()
        dec = md2text.TextDecoder(S.text_weights(0), device=dev, ctx=1024, yes_ids=(11, 222), no_ids=(55, 666))
        dec.prefill(S.activations(3, (729, 2048), "img").to(dev), S.prompt_ids(4, 64))
        dec.set_questions([S.prompt_ids(4, 32).tolist()])   # the yes/no query: 32 rows
        dec.query()
        torch.cuda.synchronize()
        log("text prefill and query tuned")
        del dec
        torch.cuda.empty_cache()
        m = trecvit.TRecViT(S.trecvit_weights(0), device=dev)
        fr = S.frames_u8(1, 16).to(dev)
        qf = (S.query_points(5, 256)[:, 1:] / 256.0).to(torch.bfloat16).to(dev)
        m.reset()
        m.step(fr[0], qf)
        m.reset()
        m.clip_state(16)
        m.forward_clip(fr, qf)
        torch.cuda.synchronize()
        log("trecvit tuned")
    fused = {k: v for k, v in ops._TUNED.items() if k not in before}
    part = {k: v for k, v in ops._TUNED_P.items() if k not in before_p}
    return fused, part


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--out", default=ops._TABLE_FILE)
    a = ap.parse_args()
    ops.MxLin.use_table = False
    log = lambda m: print(f"[tune] {m}", flush=True)
    f1, p1 = tune_tower_b1(a.reps, log)
    tune_generic(log)
    fused, part = dict(ops._TUNED), dict(ops._TUNED_P)   # every shape the forwards met (autotuned) ...
    fused.update(f1)                                     # ... with the in-context picks for the batch-1 tower
    part.update(p1)
    key = lambda k: ",".join(str(v) for v in k)
    lines = ["{", ' "note": "MI355X (gfx950) GEMM tile table: (M, N, Kw) -> (tile config, splits: > 0 in-kernel, -S = S '
                  'raw partials + mx_gemm_reduce); written by python -m strix_halo_maxx_amd.tune",']
    for name, d, last in (("fused", fused, False), ("partial", part, True)):
        items = [f'  "{key(k)}": [{v[0]}, {v[1]}]' for k, v in sorted(d.items())]
        lines += [f' "{name}": {{', ",\n".join(items), " }" + ("" if last else ",")]
    lines.append("}")
    with open(a.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    json.load(open(a.out))  # well-formed
    log(f"wrote {a.out}: {len(fused)} fused, {len(part)} partial shapes")
    return 0


if __name__ == "__main__":
    sys.exit(main())
