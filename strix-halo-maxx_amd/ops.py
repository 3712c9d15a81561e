"""Drop-in op classes over the C-ABI HIP kernels.

They keep the reference's operator protocol so the per-model forwards read like the reference's:
  * Linear:   cls(weight, bias, dtype); __call__(x, gelu=False, res=None) -> x.shape[:-1] + (N,) bf16; class flags
              fused_gelu / fused_res (moondream/gpu/md2fast.py:33-40, :55-67; hgemm.py:139-178)
  * Attention: Attn(H, T, D); __call__(q, k, v, out=None) with q, k, v (B, H, T, D) views whose last dim is
              contiguous -> (B, T, H*D) (hattn.py:17-37)
Every call launches asynchronously on torch's current stream; nothing here synchronises, so a forward made of these
calls can be captured into a HIP graph.
"""
import torch

from . import _lib
from ._lib import call, ptr, stream

BF = torch.bfloat16
ACT = {None: 0, False: 0, True: 1, "tanh": 1, "erf": 2}


def _rows(x, K):
    """2-D view (M, K) of x with unit column stride and a 16-byte aligned row stride (copies only if needed)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


class MxLin:
    """bf16 Linear on the MFMA GEMM: y = epi(x W^T + b) with epi = [GELU tanh|erf] then [+ res], torch's rounding.

    Weights stay in torch's (N, K) layout (K padded with zeros to a multiple of 8 when needed, e.g. the 588-wide patch
    embedding, whose input then comes padded from the patchify kernel). Bias is held in fp32, as the reference's
    HLin does (hgemm.py:153).
    """
    fused_gelu = True
    fused_res = True

    def __init__(self, weight, bias, dtype=BF, device="cuda"):
        assert dtype == BF, "bf16 only"
        w = weight.detach().to(device=device, dtype=BF)
        self.N, self.K = w.shape
        self.Kp = (self.K + 7) // 8 * 8
        if self.N % 4:
            raise ValueError(f"N={self.N} must be a multiple of 4")
        if self.Kp != self.K:
            wp = torch.zeros(self.N, self.Kp, device=device, dtype=BF)
            wp[:, :self.K] = w
            w = wp
        self.w = w.contiguous()
        self.b = None if bias is None else bias.detach().to(device=device, dtype=torch.float32).contiguous()
        self.cfgs = {}  # M -> tile config (None: the library's own pick)

    def __call__(self, x, gelu=False, res=None, pre=None, act=None, out=None):
        a = ACT[act if act is not None else gelu]
        x2 = _rows(x, self.K)
        if x2.shape[1] == self.K and self.Kp != self.K:
            xp = torch.zeros(x2.shape[0], self.Kp, device=x2.device, dtype=BF)
            xp[:, :self.K] = x2
            x2 = xp
        if x2.shape[1] != self.Kp:
            raise ValueError(f"input width {x2.shape[1]} != {self.K}")
        M = x2.shape[0]
        y = out if out is not None else torch.empty(M, self.N, device=x2.device, dtype=BF)
        if y.shape[-1] != self.N or y.stride(-1) != 1:
            raise ValueError("out must be (M, N) with unit column stride")
        y2 = y.view(-1, self.N) if y.dim() != 2 else y
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
        cfg = self.cfgs.get(M, -1)
        call("mx_gemm_bf16", stream(), cfg, x2.data_ptr(), x2.stride(0), self.w.data_ptr(), self.w.stride(0),
             ptr(self.b), ptr(r2), ldr, r_rows, y2.data_ptr(), y2.stride(0), M, self.N, self.Kp, a)
        return y2.view(*x.shape[:-1], self.N) if out is None else y


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


def gemm_tile(cfg):
    import ctypes
    bm, bn = ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.load().mx_gemm_cfg_tile(cfg, ctypes.byref(bm), ctypes.byref(bn)), "mx_gemm_cfg_tile")
    return bm.value, bn.value
