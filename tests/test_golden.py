"""The oracle reproduces the committed golden fixtures (tests/golden/make_golden.py): elementwise fixtures exactly,
matmul-bearing ones to rel-L2 1e-3 (CPU bf16 GEMM kernels may order fp32 sums differently across hosts)."""
import os

import torch

import oracle.md2_text as ot
import oracle.md2_vision as ov
import strix_halo_maxx_amd.synth as S
import test_oracle as T

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return torch.load(os.path.join(G, name), weights_only=True)


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_vision_block_fixture():
    f = load("vision_block.pt")
    assert rel(ov.block(f["w"], 0, f["x"], H=4), f["y"]) < 1e-3


def test_text_fixture():
    f = load("text_prefill.pt")
    m = ot.Text(f["w"], 64, S.freqs_cis(32, 256), bos=3, H=2)
    toks, lgs = m.generate(f["img"], f["prompt"], 3)
    assert toks == f["tokens"].tolist()
    assert rel(torch.stack(lgs), f["logits"]) < 1e-3


def test_ssm_fixture():
    f = load("ssm.pt")
    d = f["inputs"]
    for first in (True, False):
        z, h = T._run_ssm(d, first)
        assert rel(z, f[f"z_{int(first)}"]) < 1e-3
        assert (h - f[f"h_{int(first)}"]).abs().max() < 1e-3
