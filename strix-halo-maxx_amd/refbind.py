"""The reference-side binding of libshmaxx.so: the module a maintainer drops next to moondream/gpu/hgemm.py so that
FastMD2 runs its Linears and its vision attention on the MI355X kernels with no change to `_vision` or
`_text_layers`.

It depends on torch and the built library only (no other part of this package), binds the library with ctypes the
way the reference binds its own (moondream/gpu/hgemm.py:21-33, hattn.py:5-15), and keeps the reference's operator
protocols exactly:
  * MxLin(weight, bias, dtype); __call__(x, gelu=False, res=None); flags fused_gelu / fused_res
    (hgemm.HLin, hgemm.py:139-178; consulted by md2fast.mlp / lin_res, md2fast.py:55-67)
  * MxI8Lin(weight, bias, dtype); quant(x) -> (q, s); __call__(x, gelu=False, res=None, pre=None)
    (hgemm.HI8Lin, hgemm.py:95-137; the shared quantisation of md2fast.py:52, 174)
  * Attn(H, T, D); __call__(q, k, v, out=None) with (1, H, T, D) views whose last dim is contiguous -> (1, T, H*D)
    (hattn.Attn, hattn.py:17-37; md2fast.py:155)
  * rglru_forward(self, x, h0) -> (y, h): TAPNext's RGLRU.forward (tapnext/npu/r9/cpuemu.py:33-47), assigned the
    way the reference swaps it (`tn.RGLRU.forward = refbind.rglru_forward`, cpuemu.py:110-116)
Every call launches on torch's current stream and checks the library's status (the reference's `assert rc == 0`).
Usage in the reference: FastMD2(model, lin_cls=refbind.MxLin, tlin_cls=refbind.MxI8Lin, hattn=True) with
md2fast.HAttn = refbind.Attn (and md2fast.USE_FUSED_RES = True to run the residual adds in the GEMM epilogue).
"""
import ctypes
import os

import torch

LIB_PATH = os.environ.get("SHMAXX_LIB", os.path.join(os.path.dirname(os.path.abspath(__file__)), "libshmaxx.so"))
_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float
_ARGS = {
    "mx_gemm_bf16": [_P, _I, _I, _P, _L, _P, _L, _P, _P, _L, _I, _P, _L, _I, _I, _I, _I, _I, _I, _P, _L, _P, _L],
    "mx_sdpa": [_P, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _I, _I, _I, _I, _I, _F, _I, _I],
    "mx_quant_weight_i8": [_P, _P, _L, _P, _L, _P, _I, _I],
    "mx_quant_rows_i8": [_P, _P, _L, _P, _L, _P, _I, _I],
    "mx_gemm_i8": [_P, _I, _P, _L, _P, _L, _P, _P, _P, _P, _L, _I, _P, _L, _I, _I, _I, _I, _I, _P, _L],
    "mx_rglru_step": [_P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _L, _I, _I],
}
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build libshmaxx.so first")
        h = ctypes.CDLL(LIB_PATH)
        for name, args in _ARGS.items():
            getattr(h, name).argtypes = args
            getattr(h, name).restype = _I
        _lib = h
    return _lib


def _st():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return None if t is None else t.data_ptr()


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} returned {rc}")


class MxLin:
    """hgemm.HLin's protocol on mx_gemm_bf16: y = [GELU-tanh](x W^T + b) [+ res], torch's bf16 roundings. Weights are
    held zero-padded along K to a multiple of 64; the tile is the library's own pick (cfg = -1). A K that is not a
    multiple of 8 (the 588-wide patch embedding, where HLin falls back to F.linear, hgemm.py:155-158, 166-170) runs on
    the same kernel with the input zero-padded to the next multiple of 8."""
    fused_gelu = True
    fused_res = True
    cfg = -1

    def __init__(self, weight, bias, dtype):
        if dtype != torch.bfloat16:
            raise ValueError("bf16 only")
        w = weight.detach().to(dtype)
        self.N, self.K0 = w.shape
        if self.N % 4:
            raise ValueError(f"weight {tuple(w.shape)}: N % 4 must be 0")
        self.K = (self.K0 + 7) // 8 * 8
        self.Kw = (self.K0 + 63) // 64 * 64
        self.w = torch.zeros(self.N, self.Kw, device=w.device, dtype=dtype)
        self.w[:, :self.K0] = w
        self.b = None if bias is None else bias.detach().float().contiguous()

    def __call__(self, x, gelu=False, res=None):
        x2 = x.reshape(-1, self.K0)
        if self.K != self.K0:
            x2 = torch.nn.functional.pad(x2, (0, self.K - self.K0))
        x2 = x2.contiguous()
        M = x2.shape[0]
        c = torch.empty(M, self.N, device=x.device, dtype=torch.bfloat16)
        r = None if res is None else res.reshape(-1, self.N).contiguous()
        _ok(lib().mx_gemm_bf16(_st(), self.cfg, 1, x2.data_ptr(), self.K, self.w.data_ptr(), self.Kw, _p(self.b),
                               _p(r), self.N, 0, c.data_ptr(), self.N, M, self.N, self.K, self.Kw, int(bool(gelu)), 0,
                               None, 0, None, 0), "mx_gemm_bf16")
        return c.reshape(*x.shape[:-1], self.N)


class MxI8Lin:
    """hgemm.HI8Lin's protocol on the W8A8 kernels: per-output-channel int8 weights (round half to even, hgemm.py:
    101-106), per-token int8 activations (quant(), round half away from zero, tgemm.py:81-91), int32 accumulation,
    fp32 dequant + bias [+ GELU on the fp32 value], one bf16 rounding (i8gemm.hip:181-197) [+ res, rounded again]."""
    fused_gelu = True
    fused_res = True

    def __init__(self, weight, bias, dtype):
        w = weight.detach().to(torch.bfloat16).contiguous()
        self.N, self.K = w.shape
        if self.K % 16 or self.N % 4:
            raise ValueError(f"weight {tuple(w.shape)}: K % 16 and N % 4 must be 0")
        self.Kw = (self.K + 127) // 128 * 128
        self.wq = torch.zeros(self.N, self.Kw, device=w.device, dtype=torch.int8)
        self.sw = torch.empty(self.N, device=w.device, dtype=torch.float32)
        _ok(lib().mx_quant_weight_i8(_st(), w.data_ptr(), self.K, self.wq.data_ptr(), self.Kw, self.sw.data_ptr(),
                                     self.N, self.K), "mx_quant_weight_i8")
        self.b = None if bias is None else bias.detach().float().contiguous()

    def quant(self, x):
        x2 = x.reshape(-1, self.K).to(torch.bfloat16).contiguous()
        M = x2.shape[0]
        q = torch.empty(M, self.K, device=x.device, dtype=torch.int8)
        s = torch.empty(M, device=x.device, dtype=torch.float32)
        _ok(lib().mx_quant_rows_i8(_st(), x2.data_ptr(), self.K, q.data_ptr(), self.K, s.data_ptr(), M, self.K),
            "mx_quant_rows_i8")
        return q, s

    def __call__(self, x, gelu=False, res=None, pre=None):
        q, s = pre if pre is not None else self.quant(x)
        M = q.shape[0]
        c = torch.empty(M, self.N, device=q.device, dtype=torch.bfloat16)
        r = None if res is None else res.reshape(-1, self.N).contiguous()
        _ok(lib().mx_gemm_i8(_st(), 0, q.data_ptr(), self.K, self.wq.data_ptr(), self.Kw, s.data_ptr(),
                             self.sw.data_ptr(), _p(self.b), _p(r), self.N, 0, c.data_ptr(), self.N, M, self.N, self.K,
                             self.Kw, int(bool(gelu)), None, 0), "mx_gemm_i8")
        return c.reshape(*x.shape[:-1], self.N)


class Attn:
    """hattn.Attn's protocol on mx_sdpa: softmax(q k^T D^-0.5) v over all keys, reading q / k / v as the strided
    views the reference makes from the fused qkv output; no V^T staging buffer (the kernel transposes V in LDS)."""

    def __init__(self, H, T, D, device="cuda"):
        self.H, self.T, self.D = H, T, D

    def __call__(self, q, k, v, out=None):
        B, H, T, D = q.shape
        Tk = k.shape[2]
        if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
            raise ValueError("q, k, v need a contiguous last dimension")
        out = torch.empty(B, T, H * D, device=q.device, dtype=q.dtype) if out is None else out
        _ok(lib().mx_sdpa(_st(), q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0),
                          k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                          out.data_ptr(), out.stride(0), D, out.stride(1), B, H, T, Tk, D, D ** -0.5, 0, Tk),
            "mx_sdpa")
        return out


def rglru_forward(self, x, h0):
    """RGLRU.forward(x, h0) -> (h.to(x.dtype), h) on mx_rglru_step, for assignment to the model's RGLRU class
    (tapnext/npu/r9/cpuemu.py:33-47, swapped in at :110-116). Reads the module's input_gate.w / .b, a_gate.w / .b
    ((H, 64, 64) block-diagonal weights and (H, 64) biases) and a_param once, on the first call, and keeps their
    kernel layout on the module (the weights are frozen at inference). x: bf16 (..., C) on the GPU; h0: fp32 state of
    x's shape, or None on the first frame (then h = x * sigmoid(gate_x), returned as (bf16, fp32))."""
    prep = getattr(self, "_mx_rglru", None)
    if prep is None:
        dev = x.device
        bf = lambda t: t.detach().to(dev, torch.bfloat16).contiguous()
        prep = dict(wxT=bf(self.input_gate.w.transpose(-1, -2)), bx=bf(self.input_gate.b.reshape(-1)),
                    waT=bf(self.a_gate.w.transpose(-1, -2)), ba=bf(self.a_gate.b.reshape(-1)),
                    sp=torch.log1p(torch.exp(self.a_param.detach().double().cpu())).to(torch.bfloat16).to(dev))
        self._mx_rglru = prep
    C = prep["bx"].numel()
    x2 = x.reshape(-1, C).to(torch.bfloat16).contiguous()
    T = x2.shape[0]
    h = torch.empty(T, C, device=x2.device, dtype=torch.float32)
    y = torch.empty(T, C, device=x2.device, dtype=torch.bfloat16)
    hp = None if h0 is None else h0.reshape(T, C).float().contiguous()
    _ok(lib().mx_rglru_step(_st(), x2.data_ptr(), C, _p(hp), prep["wxT"].data_ptr(), prep["bx"].data_ptr(),
                            prep["waT"].data_ptr(), prep["ba"].data_ptr(), prep["sp"].data_ptr(), h.data_ptr(),
                            y.data_ptr(), C, T, C), "mx_rglru_step")
    return y.view(x.shape).to(x.dtype), h.view(x.shape)
