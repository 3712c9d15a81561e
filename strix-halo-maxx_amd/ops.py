"""Drop-in op classes over the C-ABI HIP kernels.

They keep the reference's operator protocol so the per-model forwards read like the reference's:
  * Linear:   cls(weight, bias, dtype); __call__(x, gelu=False, res=None) -> x.shape[:-1] + (N,) bf16; class flags
              fused_gelu / fused_res (moondream/gpu/md2fast.py:33-40, :55-67; hgemm.py:139-178)
  * Attention: Attn(H, T, D); __call__(q, k, v, out=None) with q, k, v (B, H, T, D) views whose last dim is
              contiguous -> (B, T, H*D) (hattn.py:17-37)
Every call launches asynchronously on torch's current stream; nothing here synchronises, so a forward made of these
calls can be captured into a HIP graph.
"""
import json
import os

import torch

from . import _lib
from ._lib import call, ptr, stream

BF = torch.bfloat16
ACT = {None: 0, False: 0, True: 1, "tanh": 1, "erf": 2, "glu": 3}


def _rows(x, K):
    """2-D view (M, K) of x with unit column stride and a 16-byte aligned row stride (copies only if needed)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


class Workspace:
    """Split-K scratch shared by every GEMM on one device: fp32 partial tiles + per-tile arrival counters.

    Grown on demand outside graph capture (call reserve() before capturing); counters start at zero and every
    kernel that uses them leaves them at zero. Kernels on one stream serialise, so one buffer serves all layers (as
    the reference's single split-K workspace, moondream/gpu/hgemm.py:78-83); concurrent GEMMs on two streams would
    race on it.
    """
    _by_dev = {}

    def __init__(self, device):
        self.dev = device
        self.ws = torch.empty(0, device=device, dtype=torch.float32)
        self.cnt = torch.zeros(0, device=device, dtype=torch.int32)

    @classmethod
    def get(cls, device):
        d = torch.device(device)
        key = d.index if d.index is not None else torch.cuda.current_device()
        if key not in cls._by_dev:
            cls._by_dev[key] = cls(d)
        return cls._by_dev[key]

    def reserve(self, elems, counters):
        if elems > self.ws.numel():
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("split-K workspace must be reserved before graph capture")
            self.ws = torch.empty(int(elems * 1.25) + 1024, device=self.dev, dtype=torch.float32)
        if counters > self.cnt.numel():
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("split-K counters must be reserved before graph capture")
            torch.cuda.synchronize(self.dev)
            self.cnt = torch.zeros(int(counters * 1.25) + 64, device=self.dev, dtype=torch.int32)


_TUNED = {}  # (M, N, Kw) -> (cfg, splits), shared by every layer of that shape

# Fixed tile table for MI355X (built by `python -m strix_halo_maxx_amd.tune` from in-context timings: each shape timed
# on the sequence of launches it runs in, with its real cache state). Shapes it lists skip the autotuner, so every
# process runs the same kernels; the reference's pick_cfg has the same two tiers (FIXED table, then timing,
# moondream/gpu/hgemm.py:47-76).
_TABLE_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_table_gfx950.json")


def _load_table():
    try:
        with open(_TABLE_FILE) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return {}, {}
    conv = lambda m: {tuple(int(v) for v in k.split(",")): tuple(int(v) for v in c) for k, c in m.items()}
    return conv(d.get("fused", {})), conv(d.get("partial", {}))


_FIXED, _FIXED_P = _load_table()


def _ws_need(cfg, splits, M, N):
    lib = _lib.load()
    return lib.mx_gemm_ws_elems(cfg, splits, M, N), lib.mx_gemm_ws_counters(cfg, splits, M, N)


class MxLin:
    """bf16 Linear on the MFMA GEMM: y = epi(x W^T + b) with epi = [GELU tanh|erf] then [+ res], torch's rounding.

    Weights stay in torch's (N, K) layout, zero-padded along K to a multiple of 64 (the kernel's k-step); inputs need
    K columns (K rounded up to 8: the 588-wide patch embedding takes its input zero-padded to 592 by the patchify
    kernel). Bias is held in fp32, as the reference's HLin does (hgemm.py:153). The tile config and split-K factor
    are chosen per (M, N, K) by timing every candidate once (the reference's pick_cfg autotune, hgemm.py:52-76),
    or taken from the library's default pick when tuning is off.
    """
    fused_gelu = True
    fused_res = True
    autotune = True
    use_table = True

    def __init__(self, weight, bias, dtype=BF, device="cuda"):
        assert dtype == BF, "bf16 only"
        w = weight.detach().to(device=device, dtype=BF)
        self.N, self.K0 = w.shape
        self.K = (self.K0 + 7) // 8 * 8          # input columns expected
        self.Kw = (self.K0 + 63) // 64 * 64      # padded weight row
        if self.N % 4:
            raise ValueError(f"N={self.N} must be a multiple of 4")
        if self.Kw == self.K0 and w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0:
            self.w = w  # already in the kernel's layout: share the storage (e.g. a row slice of a fused weight)
        else:
            wp = torch.zeros(self.N, self.Kw, device=device, dtype=BF)
            wp[:, :self.K0] = w
            self.w = wp
        self.Kp = self.K                         # width of the input this layer reads
        self.b = None if bias is None else bias.detach().to(device=device, dtype=torch.float32).contiguous()
        self.cfgs = {}  # M -> (cfg, splits); absent: tuned (or library pick) on first use
        self.dev = self.w.device

    def _launch(self, cfg, splits, x2, y2, M, a, r2, ldr, r_rows, ws, act_cols=0):
        """splits > 0: mx_gemm_bf16 (in-kernel split-K when > 1); splits = -S: the fence-free split-K, raw partials of
        S splits into the workspace (mx_gemm_bf16_partial) then the epilogue over their sum (mx_gemm_reduce)."""
        lib = _lib.load()
        if splits < 0:
            S, N = -splits, self.N
            if S * M * N > ws.ws.numel():
                return -3
            P = ws.ws[:S * M * N].view(S, M, N)
            rc = _partial(self, cfg, S, x2, P, M)
            if rc != 0:
                return rc
            return lib.mx_gemm_reduce(stream(), P.data_ptr(), S, M * N, N, ptr(self.b), ptr(r2), ldr, r_rows,
                                      y2.data_ptr(), y2.stride(0), M, N, a, act_cols)
        return lib.mx_gemm_bf16(
            stream(), cfg, splits, x2.data_ptr(), x2.stride(0), self.w.data_ptr(), self.w.stride(0), ptr(self.b),
            ptr(r2), ldr, r_rows, y2.data_ptr(), y2.stride(0), M, self.N, self.K, self.Kw, a, act_cols,
            ptr(ws.ws), ws.ws.numel(), ptr(ws.cnt), ws.cnt.numel())

    def _pick(self, M, x2, y2, a, r2, ldr, r_rows, ws):
        key = (M, self.N, self.Kw)
        if key in _TUNED:
            return _TUNED[key]
        if MxLin.use_table and key in _FIXED:
            _TUNED[key] = _FIXED[key]
            return _TUNED[key]
        lib = _lib.load()
        if not MxLin.autotune or torch.cuda.is_current_stream_capturing():
            p = lib.mx_gemm_pick(M, self.N, self.Kw)
            c = (p // 16, p % 16)
        else:
            c = tune_gemm(self, M, x2, y2, a, r2, ldr, r_rows, ws)
        _TUNED[key] = c
        return c

    def __call__(self, x, gelu=False, res=None, pre=None, act=None, out=None, act_cols=0):
        """act: None / "tanh" / "erf" / "glu" (gated GELU on interleaved (gate, up) weight rows: output width N / 2);
        act_cols > 0 limits the activation to output columns < act_cols."""
        a = ACT[act if act is not None else gelu]
        Nout = self.N // 2 if a == 3 else self.N
        x2 = _rows(x, self.K)
        if x2.shape[1] == self.K0 and self.K != self.K0:
            xp = torch.zeros(x2.shape[0], self.K, device=x2.device, dtype=BF)
            xp[:, :self.K0] = x2
            x2 = xp
        if x2.shape[1] != self.K:
            raise ValueError(f"input width {x2.shape[1]} != {self.K}")
        M = x2.shape[0]
        y = out if out is not None else torch.empty(M, Nout, device=x2.device, dtype=BF)
        if y.shape[-1] != Nout or y.stride(-1) != 1:
            raise ValueError("out must be (M, N) with unit column stride")
        y2 = y.view(-1, Nout) if y.dim() != 2 else y
        r2, r_rows, ldr = None, 0, 0
        if res is not None:
            r2 = res.reshape(-1, self.N)
            if r2.stride(1) != 1:
                r2 = r2.contiguous()
            ldr = r2.stride(0)
            if r2.shape[0] != M:
                if M % r2.shape[0]:
                    raise ValueError("residual rows must equal or divide the output rows")
                r_rows = r2.shape[0]
        ws = Workspace.get(x2.device)
        cfg, splits = self.cfgs.get(M) or self._pick(M, x2, y2, a, r2, ldr, r_rows, ws)
        if splits > 1:
            ws.reserve(*_ws_need(cfg, splits, M, self.N))
        elif splits < 0:
            ws.reserve(-splits * M * self.N, 0)
        _lib.check(self._launch(cfg, splits, x2, y2, M, a, r2, ldr, r_rows, ws, act_cols), "mx_gemm_bf16")
        return y2.view(*x.shape[:-1], Nout) if out is None else y

    def partial(self, x, out=None):
        """Raw fp32 split-K partial sums of x W^T, shape (splits, M, N), for a consumer that adds them in order
        together with the bias (residual_layernorm). The tile config and split count are tuned per (M, N, K)."""
        x2 = _rows(x, self.K)
        if x2.shape[1] != self.K:
            raise ValueError(f"input width {x2.shape[1]} != {self.K}")
        M = x2.shape[0]
        cfg, sp = _partial_cfg(self, M, x2)
        P = out if out is not None else torch.empty(sp, M, self.N, device=x2.device, dtype=torch.float32)
        if P.shape != (sp, M, self.N) or P.stride(2) != 1:
            raise ValueError("out must be (splits, M, N) fp32 with unit column stride")
        _lib.check(_partial(self, cfg, sp, x2, P, M), "mx_gemm_bf16_partial")
        return P

    def res_ln(self, x, res, ln, eps=1e-5, x_out=None, y_out=None):
        """x' = bf16(bf16(x W^T + b) + res) and y = LayerNorm(x'; ln = (gamma, beta)) in one launch
        (mx_gemm_bf16_res_ln): the residual Linear and the normalisation that reads its output. Only where
        res_ln_fits(M, N); returns (x', y)."""
        x2 = _rows(x, self.K)
        if x2.shape[1] != self.K:
            raise ValueError(f"input width {x2.shape[1]} != {self.K}")
        M, N = x2.shape[0], self.N
        r2 = _rows(res, N)
        X = x_out if x_out is not None else torch.empty(M, N, device=x2.device, dtype=BF)
        Y = y_out if y_out is not None else torch.empty(M, N, device=x2.device, dtype=BF)
        ws = RlnWorkspace.get(x2.device, N)
        _lib.check(_lib.load().mx_gemm_bf16_res_ln(
            stream(), x2.data_ptr(), x2.stride(0), self.w.data_ptr(), self.w.stride(0), ptr(self.b), r2.data_ptr(),
            r2.stride(0), X.data_ptr(), X.stride(0), ln[0].data_ptr(), ln[1].data_ptr(), Y.data_ptr(), Y.stride(0), M,
            N, self.K, self.Kw, float(eps), ws.stats.data_ptr(), ws.stats.numel(), ws.sync.data_ptr(),
            ws.sync.numel()), "mx_gemm_bf16_res_ln")
        return X, Y

    def res_rms(self, x, res, sc1, eps=1e-6, x_out=None, y_out=None):
        """x' = bf16(bf16(x W^T + b) + res) and y = the TRecViT RMSNorm of x' (sc1 = bf16(scale + 1)) in one launch
        (mx_gemm_bf16_res_rms). Only where res_ln_fits(M, N); returns (x', y)."""
        x2 = _rows(x, self.K)
        if x2.shape[1] != self.K:
            raise ValueError(f"input width {x2.shape[1]} != {self.K}")
        M, N = x2.shape[0], self.N
        r2 = _rows(res, N)
        X = x_out if x_out is not None else torch.empty(M, N, device=x2.device, dtype=BF)
        Y = y_out if y_out is not None else torch.empty(M, N, device=x2.device, dtype=BF)
        ws = RlnWorkspace.get(x2.device, N)
        _lib.check(_lib.load().mx_gemm_bf16_res_rms(
            stream(), x2.data_ptr(), x2.stride(0), self.w.data_ptr(), self.w.stride(0), ptr(self.b), r2.data_ptr(),
            r2.stride(0), X.data_ptr(), X.stride(0), sc1.data_ptr(), Y.data_ptr(), Y.stride(0), M, N, self.K, self.Kw,
            float(eps), ws.stats.data_ptr(), ws.stats.numel(), ws.sync.data_ptr(), ws.sync.numel()),
            "mx_gemm_bf16_res_rms")
        return X, Y


_TUNED_P = {}  # (M, N, Kw) -> (cfg, splits) of the split-K partial GEMM


def _partial(lin, cfg, sp, x2, P, M):
    return _lib.load().mx_gemm_bf16_partial(stream(), cfg, sp, x2.data_ptr(), x2.stride(0), lin.w.data_ptr(),
                                            lin.w.stride(0), P.data_ptr(), P.stride(1), P.stride(0), M, lin.N, lin.K,
                                            lin.Kw)


def has_partial_pick(M, lin):
    """Whether the split-K partial GEMM of (M, lin.N, lin.Kw) has a pick already (tuned in this process or in the
    fixed table), so that a caller under graph capture does not fall back to the untuned default."""
    key = (M, lin.N, lin.Kw)
    return key in _TUNED_P or (MxLin.use_table and key in _FIXED_P)


def _partial_cfg(lin, M, x2):
    """(cfg, splits) for the split-K partial GEMM: every config with a partial-sum mode x splits in 1..4 timed once on
    the real operands (outside graph capture), else 64x64 tiles with 2 splits."""
    key = (M, lin.N, lin.Kw)
    if key in _TUNED_P:
        return _TUNED_P[key]
    if MxLin.use_table and key in _FIXED_P:
        _TUNED_P[key] = _FIXED_P[key]
        return _TUNED_P[key]
    lib = _lib.load()
    best = (8, 2)
    if MxLin.autotune and not torch.cuda.is_current_stream_capturing():
        nk = lin.Kw // 64
        bt = float("inf")
        P = torch.empty(4, M, lin.N, device=x2.device, dtype=torch.float32)
        for cfg in range(lib.mx_gemm_ncfg()):
            for sp in (1, 2, 3, 4):
                if sp > 1 and (nk // sp < 2 or (sp - 1) * (-(-nk // sp)) >= nk):
                    continue
                run = lambda: _partial(lin, cfg, sp, x2, P, M)
                if run() != 0:
                    continue
                run()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(10):
                    run()
                e1.record()
                e1.synchronize()
                t = e0.elapsed_time(e1)
                if t < bt:
                    best, bt = (cfg, sp), t
        del P
    _TUNED_P[key] = best
    return best


def tune_gemm(lin, M, x2, y2, a, r2, ldr, r_rows, ws, reps=10):
    """Time every (tile config, split-K) candidate on the real operands; return the fastest. Runs eagerly on the
    current stream (writes y2, which the caller overwrites right after)."""
    lib = _lib.load()
    cands = []
    nk = lin.Kw // 64
    for cfg in range(lib.mx_gemm_ncfg()):
        for sp in ((1, 2, 3, 4, 6, 8) if tune_gemm.split_k else (1,)):
            if sp > 1 and (nk // sp < 3 or (sp - 1) * (-(-nk // sp)) >= nk):
                continue
            cands.append((cfg, sp))
        if tune_gemm.partial and a != 3:
            for sp in (2, 4, 8, 16):
                if nk // sp < 2 or (sp - 1) * (-(-nk // sp)) >= nk:
                    continue
                cands.append((cfg, -sp))
    best, bt = None, float("inf")
    for cfg, sp in cands:
        if sp > 1:
            ws.reserve(*_ws_need(cfg, sp, M, lin.N))
        elif sp < 0:
            ws.reserve(-sp * M * lin.N, 0)
        run = lambda: lin._launch(cfg, sp, x2, y2, M, a, r2, ldr, r_rows, ws)
        if run() != 0:
            continue
        run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        e1.synchronize()
        t = e0.elapsed_time(e1)
        if t < bt:
            best, bt = (cfg, sp), t
    return best


# Split-K candidates in the tuner: off by default (the cross-XCD release fence of the last-arriver reduction costs
# more than the extra parallelism buys at these shapes; the path stays available and tested).
tune_gemm.split_k = False
# Fence-free split-K candidates (partial GEMM + mx_gemm_reduce, pick (cfg, -S)): on by default; they win where the
# grid of output tiles is far below the 256 CUs (the 32 / 64-row prompt and query GEMMs).
tune_gemm.partial = True


class MxI8Lin:
    """W8A8 Linear (the reference's HI8Lin, moondream/gpu/hgemm.py:95-137): int8 weights with a per-output-channel scale
    (amax / 127, round half to even, hgemm.py:101-106), int8 activations with a per-token dynamic scale (quant(),
    tgemm.py:81-91), int32 MFMA accumulation, fp32 dequant ((acc * s_x) * s_w) + bias, GELU-tanh on that fp32 value
    when asked (fused_gelu), one bf16 rounding (i8gemm.hip:181-197). `pre` takes an already quantised input (q, s),
    so layers that read the same activation share one quantisation (md2fast.py:52, 174). A residual is added to the
    rounded output and rounded again, exactly the reference's separate bf16 add (lin_res / mlp, md2fast.py:55-67),
    so the class also offers fused_res.
    Weights are zero-padded along K to a multiple of 128 (the int8 k-step); K must be a multiple of 16.
    """
    fused_gelu = True
    fused_res = True

    def __init__(self, weight, bias, dtype=BF, device="cuda"):
        assert dtype == BF, "bf16 activations only"
        w = weight.detach().to(device=device, dtype=BF)
        self.N, self.K = w.shape
        if self.K % 16 or self.N % 4:
            raise ValueError(f"W8A8 Linear needs K % 16 == 0 and N % 4 == 0, got {tuple(w.shape)}")
        self.Kw = (self.K + 127) // 128 * 128
        self.wq, self.sw = self.quantize_weight(w, self.Kw)
        self.b = None if bias is None else bias.detach().to(device=w.device, dtype=torch.float32).contiguous()
        self.cfgs = {}
        self.dev = w.device

    @classmethod
    def from_quantized(cls, wq, sw, bias):
        """A Linear over already quantised weights (int8 (N, Kw) with Kw % 128 == 0 and zeros past K = Kw, fp32 (N,)
        scales): row slices of a fused quantised weight share its storage."""
        self = cls.__new__(cls)
        self.N, self.Kw = wq.shape
        self.K = self.Kw
        if self.Kw % 128 or wq.stride(1) != 1 or wq.stride(0) % 16:
            raise ValueError("quantised weight rows must be contiguous, 16-byte aligned, a multiple of 128 wide")
        self.wq, self.sw = wq, sw
        self.b = None if bias is None else bias.detach().to(device=wq.device, dtype=torch.float32).contiguous()
        self.cfgs = {}
        self.dev = wq.device
        return self

    @staticmethod
    def quantize_weight(weight, Kw=None):
        """(N, K) bf16 weight (on the device) -> int8 (N, Kw) zero-padded past K, fp32 (N,) per-row scale
        (hgemm.py:101-106), by the library's quantisation kernel."""
        w = weight.detach().to(dtype=BF).contiguous()
        N, K = w.shape
        Kw = K if Kw is None else Kw
        q = torch.zeros(N, Kw, device=w.device, dtype=torch.int8)
        s = torch.empty(N, device=w.device, dtype=torch.float32)
        call("mx_quant_weight_i8", stream(), w.data_ptr(), w.stride(0), q.data_ptr(), q.stride(0), s.data_ptr(), N, K)
        return q, s

    def quant(self, x):
        """Per-token int8 quantisation of x (..., K) -> (q (M, K) int8, s (M,) fp32)."""
        x2 = _rows(x, self.K)
        M = x2.shape[0]
        q = torch.empty(M, self.K, device=x2.device, dtype=torch.int8)
        sc = torch.empty(M, device=x2.device, dtype=torch.float32)
        call("mx_quant_rows_i8", stream(), x2.data_ptr(), x2.stride(0), q.data_ptr(), q.stride(0), sc.data_ptr(), M,
             self.K)
        return q, sc

    def _launch(self, cfg, q, sc, y2, M, a, r2, ldr, r_rows, P=None, splits=1):
        """splits = -S: raw int32 partials of S splits into the workspace (mx_gemm_i8_partial), then the W8A8
        epilogue over their exact sum (mx_gemm_i8_reduce): equal to the one-launch GEMM bit for bit."""
        lib = _lib.load()
        if splits < 0:
            S, N = -splits, self.N
            ws = Workspace.get(q.device)
            if S * M * N > ws.ws.numel():
                return -3
            Pw = ws.ws[:S * M * N].view(torch.int32).view(S, M, N)
            rc = lib.mx_gemm_i8_partial(stream(), cfg, S, q.data_ptr(), q.stride(0), self.wq.data_ptr(),
                                        self.wq.stride(0), Pw.data_ptr(), N, M * N, M, N, self.K, self.Kw)
            if rc != 0:
                return rc
            return lib.mx_gemm_i8_reduce(stream(), Pw.data_ptr(), S, M * N, N, ptr(sc), self.sw.data_ptr(),
                                         ptr(self.b), ptr(r2), ldr, r_rows, y2.data_ptr(), y2.stride(0), M, N, a)
        return lib.mx_gemm_i8(stream(), cfg, q.data_ptr(), q.stride(0), self.wq.data_ptr(), self.wq.stride(0),
                              ptr(sc), self.sw.data_ptr(), ptr(self.b), ptr(r2), ldr, r_rows, ptr(y2),
                              y2.stride(0) if y2 is not None else 0, M, self.N, self.K, self.Kw, a, ptr(P),
                              P.stride(0) if P is not None else 0)

    def _pick(self, M, q, sc, y2):
        """(cfg, splits) for this M: every kind-0 tile config in one launch, and with raw partials over 2 / 4 / 8 / 16
        k-splits plus the reduction, each timed on the real operands (outside graph capture)."""
        key = ("i8", M, self.N, self.Kw)
        if key in _TUNED:
            return _TUNED[key]
        best = (0, 1)
        if MxLin.autotune and not torch.cuda.is_current_stream_capturing():
            bt = float("inf")
            nk = self.Kw // 128
            ws = Workspace.get(q.device)
            cands = [(c, 1) for c in range(_lib.load().mx_gemm_ncfg()) if _lib.load().mx_gemm_cfg_kind(c) == 0]
            if tune_gemm.partial:
                cands += [(c, -sp) for c, _ in list(cands) for sp in (2, 4, 8, 16)
                          if nk // sp >= 2 and (sp - 1) * (-(-nk // sp)) < nk]
            for cfg, sp in cands:
                if sp < 0:
                    ws.reserve(-sp * M * self.N, 0)
                run = lambda: self._launch(cfg, q, sc, y2, M, 0, None, 0, 0, splits=sp)
                if run() != 0:
                    continue
                run()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(5):
                    run()
                e1.record()
                e1.synchronize()
                t = e0.elapsed_time(e1)
                if t < bt:
                    best, bt = (cfg, sp), t
        _TUNED[key] = best
        return best

    def __call__(self, x, gelu=False, res=None, pre=None, act=None, out=None):
        a = ACT[act if act is not None else gelu]
        if a == 3:
            raise ValueError("no gated GELU in the W8A8 path")
        q, sc = pre if pre is not None else self.quant(x)
        M = q.shape[0]
        y = out if out is not None else torch.empty(M, self.N, device=q.device, dtype=BF)
        y2 = y.view(-1, self.N) if y.dim() != 2 else y
        r2, r_rows, ldr = None, 0, 0
        if res is not None:
            r2 = res.reshape(-1, self.N)
            if r2.stride(1) != 1:
                r2 = r2.contiguous()
            ldr = r2.stride(0)
            if r2.shape[0] != M:
                raise ValueError("residual rows must equal the output rows")
        cfg = self.cfgs.get(M)
        if cfg is None:
            cfg = self.cfgs[M] = self._pick(M, q, sc, y2)
        cfg, splits = cfg if isinstance(cfg, tuple) else (cfg, 1)
        if splits < 0:
            Workspace.get(q.device).reserve(-splits * M * self.N, 0)
        _lib.check(self._launch(cfg, q, sc, y2, M, a, r2, ldr, r_rows, splits=splits), "mx_gemm_i8")
        return y2.view(*x.shape[:-1], self.N) if out is None else y

    def acc_i32(self, q, cfg=0):
        """Raw int32 accumulators q Wq^T (M, N) (parity checks)."""
        M = q.shape[0]
        P = torch.empty(M, self.N, device=q.device, dtype=torch.int32)
        _lib.check(self._launch(cfg, q, None, None, M, 0, None, 0, 0, P=P), "mx_gemm_i8")
        return P


def sdpa(q, k, v, out=None, scale=None, qpos0=0, causal_from=None):
    """Fused attention. q (B, H, Tq, D), k/v (B, H, Tk, D) strided views (unit stride on D); out (B, Tq, H*D).

    Mask: key j is visible to query i iff j < Tk and (j < causal_from or j <= qpos0 + i); causal_from=None = no mask.
    """
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if out is None:
        out = torch.empty(B, Tq, H * D, device=q.device, dtype=BF)
    sc = D ** -0.5 if scale is None else scale
    cf = Tk if causal_from is None else causal_from
    call("mx_sdpa", stream(), q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
         k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
         out.data_ptr(), out.stride(0), D, out.stride(1), B, H, Tq, Tk, D, float(sc), int(qpos0), int(cf))
    return out


def sdpa_tiling(B, H, Tq, D):
    """(query waves, key waves, keys per staged block, ring stages) of the kernel sdpa runs for this problem."""
    import ctypes
    t = (ctypes.c_int * 4)()
    _lib.load().mx_sdpa_tiling(B, H, Tq, D, ctypes.cast(t, ctypes.c_void_p))
    return tuple(t)


def sdpa_symbol(B, H, Tq, D):
    """The attention kernel's name as rocprofv3 prints it."""
    return "attn_fwd_kernel<{}, {}>".format(D, ", ".join(str(v) for v in sdpa_tiling(B, H, Tq, D)))


class Attn:
    """Reference protocol (hattn.py:17-37): Attn(H, T, D)(q, k, v) -> (B, T, H*D). No V^T staging buffer is needed:
    the kernel transposes V through LDS."""

    def __init__(self, H, T, D, device="cuda", scale=None):
        self.H, self.T, self.D = H, T, D
        self.scale = D ** -0.5 if scale is None else scale

    def __call__(self, q, k, v, out=None):
        return sdpa(q, k, v, out=out, scale=self.scale)


def layernorm(x, w, b, eps=1e-5, out=None):
    D = x.shape[-1]
    x2 = _rows(x, D)
    y = out if out is not None else torch.empty(x2.shape, device=x.device, dtype=BF)
    call("mx_layernorm", stream(), x2.data_ptr(), x2.stride(0), w.data_ptr(), b.data_ptr(), y.data_ptr(),
         y.reshape(-1, D).stride(0), x2.shape[0], D, float(eps))
    return y.view(*x.shape) if out is None else y


class RlnWorkspace:
    """Row statistics and their generation counters for mx_gemm_bf16_res_ln / _res_rms, one per (device, N), allocated
    zeroed once at their largest size (the launch allows at most one 64 x 64 tile per CU, so at most 256 tiles: 256
    x 128 stats words; 1 + 2 x 256 sync words) and then owned by the kernel, which leaves them ready for the next
    call. Keyed by N because where a row block's statistics sit depends on the tiles per row block (N / 64): calls
    of another N on the same words could meet old words that carry the epoch they expect. Calls of one N may have
    any M. Calls on one stream serialise; two streams must not share them."""
    _by_key = {}

    def __init__(self, device):
        self.stats = torch.zeros(256 * 128, device=device, dtype=torch.int64)
        self.sync = torch.zeros(1024, device=device, dtype=torch.int32)

    @staticmethod
    def _dev_index(device):
        d = torch.device(device)
        return d.index if d.index is not None else torch.cuda.current_device()

    @classmethod
    def get(cls, device, N):
        key = (cls._dev_index(device), int(N))
        if key not in cls._by_key:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("the residual-LayerNorm workspace must exist before graph capture")
            cls._by_key[key] = cls(torch.device(device))
        return cls._by_key[key]

    @classmethod
    def device_error(cls, device):
        """Non-zero if a wait of any fused residual-LayerNorm GEMM on the device timed out (its results are then
        undefined). Synchronises."""
        i = cls._dev_index(device)
        return max((ws.error() for (d, _), ws in cls._by_key.items() if d == i), default=0)

    @classmethod
    def reset_device(cls, device):
        """Zero every workspace of the device (after a timed-out wait)."""
        i = cls._dev_index(device)
        for (d, _), ws in cls._by_key.items():
            if d == i:
                ws.reset()

    def error(self):
        """Non-zero if a wait of a fused residual-LayerNorm GEMM on these words timed out."""
        return int(self.sync[0].item())

    def reset(self):
        """Zero both buffers (after a timed-out wait, before the next call)."""
        self.stats.zero_()
        self.sync.zero_()


def _cu_count(device):
    return torch.cuda.get_device_properties(torch.device(device)).multi_processor_count


def res_ln_fits(M, N, device):
    """mx_gemm_bf16_res_ln's shape rule: N a multiple of 64 (at most 4096) and one 64 x 64 tile per CU at most."""
    return N % 64 == 0 and N <= 4096 and ((M + 63) // 64) * (N // 64) <= _cu_count(device)


def residual_layernorm(P, bias, res, ln=None, eps=1e-5, x_out=None, y_out=None):
    """Reduce split-K partials P (splits, M, D) fp32: x = bf16(bf16(sum P + bias) + res); y = LayerNorm(x; ln) when
    ln = (gamma, beta) is given. Returns (x, y) (y None without ln)."""
    S, M, D = P.shape
    r2 = _rows(res, D)
    x = x_out if x_out is not None else torch.empty(M, D, device=P.device, dtype=BF)
    y = None
    if ln is not None:
        y = y_out if y_out is not None else torch.empty(M, D, device=P.device, dtype=BF)
    call("mx_residual_layernorm", stream(), P.data_ptr(), S, P.stride(0), P.stride(1), ptr(bias), r2.data_ptr(),
         r2.stride(0), x.data_ptr(), x.stride(0), ptr(ln[0]) if ln else None, ptr(ln[1]) if ln else None, ptr(y),
         y.stride(0) if y is not None else 0, M, D, float(eps))
    return x, y


def residual_rmsnorm(P, bias, res, sc1, eps=1e-6, x_out=None, y_out=None):
    """Reduce split-K partials P (splits, M, D) fp32: x = bf16(bf16(sum P + bias) + res); y = the TRecViT RMSNorm of
    x with sc1 = bf16(scale + 1). Returns (x, y)."""
    S, M, D = P.shape
    r2 = _rows(res, D)
    x = x_out if x_out is not None else torch.empty(M, D, device=P.device, dtype=BF)
    y = y_out if y_out is not None else torch.empty(M, D, device=P.device, dtype=BF)
    call("mx_residual_rmsnorm", stream(), P.data_ptr(), S, P.stride(0), P.stride(1), ptr(bias), r2.data_ptr(),
         r2.stride(0), x.data_ptr(), x.stride(0), sc1.data_ptr(), y.data_ptr(), y.stride(0), M, D, float(eps))
    return x, y


def rmsnorm(x, sc1, eps=1e-6, out=None):
    """TRecViT RMSNorm; sc1 = bf16(scale + 1)."""
    D = x.shape[-1]
    x2 = _rows(x, D)
    y = out if out is not None else torch.empty(x2.shape, device=x.device, dtype=BF)
    call("mx_rmsnorm", stream(), x2.data_ptr(), x2.stride(0), sc1.data_ptr(), y.data_ptr(),
         y.reshape(-1, D).stride(0), x2.shape[0], D, float(eps))
    return y.view(*x.shape) if out is None else y


def patchify(img_u8, patch, mode, ldo=None, out=None):
    """(B, S, S, 3) u8 -> (B * (S/P)^2, ldo) bf16 patch rows, (c, ky, kx) column order, zero padded to ldo."""
    B, S, _, _ = img_u8.shape
    K = 3 * patch * patch
    ldo = (K + 7) // 8 * 8 if ldo is None else ldo
    G = S // patch
    y = out if out is not None else torch.empty(B * G * G, ldo, device=img_u8.device, dtype=BF)
    call("mx_patchify_u8", stream(), img_u8.data_ptr(), y.data_ptr(), ldo, B, S, patch, mode)
    return y


def resize_patchify(img_u8, size, patch, ldo=None, out=None):
    """(B, Hs, Ws, 3) u8 -> bilinear resize to size x size, / 127.5 - 1, as (B * (size/P)^2, ldo) bf16 patch rows
    (the TRecViT preprocess, tapnext/npu/step8.py:379-383, fused with the patch-conv input)."""
    B, Hs, Ws, _ = img_u8.shape
    K = 3 * patch * patch
    ldo = (K + 7) // 8 * 8 if ldo is None else ldo
    G = size // patch
    y = out if out is not None else torch.empty(B * G * G, ldo, device=img_u8.device, dtype=BF)
    call("mx_resize_patchify_u8", stream(), img_u8.data_ptr(), Hs, Ws, y.data_ptr(), ldo, B, size, patch)
    return y


def gemm_tile(cfg):
    import ctypes
    bm, bn = ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.load().mx_gemm_cfg_tile(cfg, ctypes.byref(bm), ctypes.byref(bn)), "mx_gemm_cfg_tile")
    return bm.value, bn.value
