"""C ABI checks that run without a GPU: the library loads, exports every entry point include/shmaxx.h declares, and
its host-side validation rejects the shapes / layouts / configs the kernels do not support (the reference's
negative status codes, moondream/gpu/hip/i8gemm.hip:481-482, :535, :557-561; attn.hip:435-440). No kernel is
launched here: every call below is refused before any HIP API call."""
import ctypes
import os
import re

import pytest
import torch

from strix_halo_maxx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "shmaxx.h")
A16 = 0x10000  # fake 16-byte aligned device addresses: validation never dereferences them


def declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|long|void)\s+(mx_\w+)\s*\(", src, re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert len(names) >= 20
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for n in declared():
        assert hasattr(lib, n), n
    # and the binding declares nothing the header does not
    assert set(_lib.SIGNATURES) <= set(declared())


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.MxError):
        _lib.load()


def gemm_check(**kw):
    a = dict(cfg=0, splits=1, A=A16, lda=1152, W=A16, ldw=1152, bias=A16, R=None, ldr=0, C=A16, ldc=1152, M=729,
             N=1152, K=1152, Kw=1152, act=0, ws=None, ws_elems=0, cnt=None, n_cnt=0)
    a.update(kw)
    return _lib.load().mx_gemm_check(*a.values())


def test_gemm_validation():
    assert gemm_check() == 0
    assert gemm_check(K=1150, lda=1150) == -2          # K not a multiple of 8
    assert gemm_check(Kw=1100) == -2                    # weight row not a multiple of the 64-wide k-step
    assert gemm_check(N=1150, ldc=1152) == -2           # N not a multiple of 4
    assert gemm_check(A=A16 + 2) == -4                  # A not 16-byte aligned
    assert gemm_check(C=A16 + 2) == -4
    assert gemm_check(act=4) == -1
    assert gemm_check(cfg=99) == -1
    assert gemm_check(A=None) == -6
    assert gemm_check(act=3, R=A16, ldr=1152) == -1     # gated GELU has no residual
    assert gemm_check(act=3, ldc=576) == 0              # gated GELU writes N / 2 columns
    assert gemm_check(splits=4) == -6                   # split-K needs a workspace
    need = _lib.load().mx_gemm_ws_elems(0, 4, 729, 1152)
    ncnt = _lib.load().mx_gemm_ws_counters(0, 4, 729, 1152)
    assert need == 6 * 9 * 4 * 128 * 128 and ncnt == 54
    assert gemm_check(splits=4, ws=A16, ws_elems=need, cnt=A16, n_cnt=ncnt) == 0
    assert gemm_check(splits=4, ws=A16, ws_elems=need - 1, cnt=A16, n_cnt=ncnt) == -3
    assert gemm_check(splits=18, ws=A16, ws_elems=10 ** 9, cnt=A16, n_cnt=10 ** 6) == 0
    assert gemm_check(splits=17, ws=A16, ws_elems=10 ** 9, cnt=A16, n_cnt=10 ** 6) == -3  # an empty split


def test_gemm_entry_point_refuses_before_launch():
    lib = _lib.load()
    rc = lib.mx_gemm_bf16(None, 0, 1, A16, 1150, A16, 1152, None, None, 0, 0, A16, 1152, 729, 1152, 1150, 1152, 0, 0,
                          None, 0, None, 0)
    assert rc == -2


def test_gemm_pick_is_a_valid_config():
    lib = _lib.load()
    for M, N, K in [(729, 3456, 1152), (729, 1152, 4352), (186624, 4304, 1152), (1, 6144, 2048)]:
        p = lib.mx_gemm_pick(M, N, K)
        cfg, sp = p // 16, p % 16
        assert 0 <= cfg < lib.mx_gemm_ncfg() and sp >= 1
        bm, bn = ctypes.c_int(), ctypes.c_int()
        assert lib.mx_gemm_cfg_tile(cfg, ctypes.byref(bm), ctypes.byref(bn)) == 0
        assert bm.value % 32 == 0 and bn.value % 32 == 0 and 32 <= min(bm.value, bn.value) and max(bm.value, bn.value) <= 256
        assert lib.mx_gemm_cfg_kind(cfg) in (0, 1)
        assert sp == 1 or lib.mx_gemm_cfg_kind(cfg) == 0
    assert lib.mx_gemm_cfg_kind(lib.mx_gemm_ncfg()) == -1 and lib.mx_gemm_cfg_kind(-1) == -1


def test_sdpa_validation():
    lib = _lib.load()
    ok = lambda **kw: lib.mx_sdpa_check(*dict(dict(Q=A16, sq_t=3456, K=A16, sk_t=3456, V=A16, sv_t=3456, O=A16,
                                                   so_t=1152, B=1, H=16, Tq=729, Tk=729, D=72), **kw).values())
    assert ok() == 0
    assert ok(D=80) == -1          # head dims 64 and 72 only (the reference's DP table, hattn.py:21)
    assert ok(sq_t=3455) == -2
    assert ok(K=A16 + 8) == -4
    assert ok(Tk=0) == -2
    rc = lib.mx_sdpa(None, A16, 0, 72, 3456, A16, 0, 72, 3456, A16, 0, 72, 3456, A16, 0, 72, 1152, 1, 16, 729, 729, 80,
                     0.1, 0, 729)
    assert rc == -1


def test_sdpa_tiling_pick():
    """The tiling table (host-side, no launch): every pick is a tiling mx_sdpa instantiates."""
    import strix_halo_maxx_amd.ops as ops
    assert ops.sdpa_tiling(1, 16, 729, 72) == (2, 4, 128, 2)      # vision tower, batch 1
    assert ops.sdpa_tiling(13, 16, 729, 72) == (4, 2, 64, 4)      # batch 13 / 256
    assert ops.sdpa_tiling(1, 32, 64, 64) == (1, 4, 128, 2)       # 64-token prompt
    assert ops.sdpa_tiling(1, 32, 730, 64) == (4, 4, 128, 2)      # text prefix
    assert ops.sdpa_tiling(1, 12, 1280, 64) == (2, 8, 256, 2)     # TRecViT
    assert ops.sdpa_tiling(16, 12, 1280, 64) == (4, 1, 64, 3)     # TRecViT clip
    assert ops.sdpa_symbol(1, 16, 729, 72) == "attn_fwd_kernel<72, 2, 4, 128, 2>"


def test_other_entry_points_refuse_bad_shapes():
    lib = _lib.load()
    assert lib.mx_layernorm(None, A16, 1152, A16, A16, A16, 1152, 729, 1150, 1e-5) == -2
    assert lib.mx_rmsnorm(None, A16 + 4, 768, A16, A16, 768, 10, 768, 1e-6) == -4
    assert lib.mx_patchify_u8(None, A16, A16, 500, 1, 378, 14, 0) == -2          # ldo < 588
    assert lib.mx_resize_patchify_u8(None, A16, 480, 854, A16, 190, 1, 256, 8) == -2  # ldo < 192
    assert lib.mx_resize_patchify_u8(None, A16, 0, 854, A16, 192, 1, 256, 8) == -2    # empty source
    assert lib.mx_resize_patchify_u8(None, A16, 480, 854, A16, 192, 1, 250, 8) == -2  # S % P
    assert lib.mx_resize_patchify_u8(None, None, 480, 854, A16, 192, 1, 256, 8) == -6
    assert lib.mx_rope_kv(None, A16, 6144, A16, A16, A16, A16, 1, 100, 32, 1024, 1000, 1, 0) == -2  # pos past ctx
    assert lib.mx_ln_gemv2(None, A16, A16, A16, 1e-5, A16, 2048, A16, 100, 3000, 50, A16, A16, 1) == -2  # K
    assert lib.mx_ln_gemv_argmax(None, A16, A16, A16, 1e-5, A16, 2048, A16, 51200, 2048, None, A16, 10) == -3
    assert lib.mx_decode_attn(None, A16, A16, A16, A16, 0, 1024, A16, 8, 0.125, A16, A16, A16) == -2   # H < 1
    assert lib.mx_decode_attn(None, A16, A16, A16, A16, 32, 1024, A16, 8, 0.125, None, None, None) == -6
    af = lambda H=32, K2=8192, g=A16, y2=A16, S=1, part=None, a=A16: lib.mx_decode_attn_fc2(
        None, A16, A16, A16, A16, H, 1024, A16, 0.125, S, part, a, g, A16, A16, K2, y2, 2048)
    assert af(H=0) == -2 and af(K2=4000) == -2 and af(g=A16 + 2) == -4 and af(y2=None) == -6
    assert af(S=9, part=A16) == -2 and af(S=0) == -2 and af(S=2) == -6 and af(a=None) == -6  # S, part / attn_out
    af8 = lambda K2=8192, sw=A16: lib.mx_decode_attn_fc2_i8(None, A16, A16, A16, A16, 32, 1024, A16, 0.125, 1, None,
                                                            A16, A16, A16, sw, A16, K2, A16, 2048)
    assert af8(K2=2048) == -2 and af8(sw=None) == -6
    assert lib.mx_gemv_res2(None, A16, A16, 1, None, A16, A16, 3000, A16, A16, 2048) == -2           # Kp
    assert lib.mx_gemv_res2(None, A16, A16 + 8, 1, None, A16, A16, 2048, A16, A16, 2048) == -4
    assert lib.mx_gemv_res2(None, A16, None, 4, None, A16, A16, 2048, A16, A16, 2048) == -6          # no records
    assert lib.mx_gemv_res2_i8(None, A16, A16, 1, None, A16, None, A16, 2048, A16, A16, 2048) == -6
    assert lib.mx_gemv_res2_i8(None, A16, A16, 1, None, A16, A16, A16, 2048, A16, A16, 0) == -2
    assert lib.mx_residual_layernorm(None, A16, 5, 0, 1152, None, A16, 1152, A16, 1152, None, None, None, 0,
                                     729, 1152, 1e-6) == -2                       # more than 4 splits
    assert lib.mx_gemm_bf16_partial(None, 15, 2, A16, 1152, A16, 1152, A16, 1152, 729 * 1152, 729, 1152,
                                    1152, 1152) == -1                            # an 8-wave cfg
    assert lib.mx_ssm_step(None, A16, A16, A16, A16, 1536, A16, 1536, A16, A16, A16, A16, A16, A16, A16, A16, A16,
                           A16, 768, 1280, 700) == -2                                 # C not a multiple of 64
    assert lib.mx_rglru_scan(None, A16, A16, A16, 4, 1280, 700, A16, 1536, 0, A16, 768, 0) == -2
    ssr = lambda T=512, srows=1280, rows=A16, stamps=A16, xsave=A16: lib.mx_ssm_step_rows(
        None, A16, A16, A16, A16, 1536, A16, 1536, A16, A16, A16, A16, A16, A16, A16, A16, A16, A16, 768, T, 768,
        rows, stamps, srows, xsave, 1536)
    assert ssr(T=1300) == -2           # more tokens than state rows
    assert ssr(rows=None) == -6 and ssr(stamps=None) == -6 and ssr(xsave=None) == -6
    assert lib.mx_counter_add(None, None, 1) == -6
    rd = lambda **kw: lib.mx_gemm_reduce(*(lambda a: (a.update(kw), list(a.values()))[1])(dict(
        st=None, P=A16, ns=4, ps=64 * 2048, ldp=2048, bias=None, R=None, ldr=0, rr=0, C=A16, ldc=2048, M=64,
        N=2048, act=0, an=0)))
    assert rd(N=2046, ldp=2046, ldc=2046) == -2   # N % 4
    assert rd(ps=100) == -2                       # split stride under M * ldp
    assert rd(act=4) == -2
    assert rd(act=3, R=A16, ldr=2048) == -2       # no residual with the gated GELU
    assert rd(P=A16 + 4) == -4                    # P not 16-byte aligned
    assert rd(C=None) == -6
    assert lib.mx_gemm_i8_partial(None, 8, 2, A16, 2048, A16, 2048, A16, 2048, 64 * 2048, 64, 2048, 2048,
                                  2048) == -1     # kind-1 config
    assert lib.mx_gemm_i8_partial(None, 0, 17, A16, 2048, A16, 2048, A16, 2048, 64 * 2048, 64, 2048, 2048,
                                  2048) == -3     # more splits than 128-wide k-steps
    assert lib.mx_gemm_i8_partial(None, 0, 2, A16, 2048, A16, 2048, A16, 2048, 100, 64, 2048, 2048, 2048) == -4
    assert lib.mx_gemm_i8_reduce(None, A16, 2, 64 * 2048, 2048, A16, A16, None, None, 0, 0, A16, 2048, 64, 2048,
                                 3) == -2         # no gated GELU in W8A8
    assert lib.mx_gemm_i8_reduce(None, A16, 2, 64 * 2048, 2048, None, A16, None, None, 0, 0, A16, 2048, 64, 2048,
                                 0) == -6
    # residual Linear + LayerNorm / RMSNorm in one launch (refused before the device query)
    rl = lambda **kw: lib.mx_gemm_bf16_res_ln(*{**dict(
        st=None, A=A16, lda=768, W=A16, ldw=768, bias=A16, R=A16, ldr=768, X=A16, ldx=768, g=A16, b=A16, Y=A16,
        ldy=768, M=1280, N=768, K=768, Kw=768, eps=1e-6, stats=A16, sw=1 << 20, sync=A16, syw=1 << 10), **kw}.values())
    assert rl(b=None) == -6 and rl(R=None) == -6 and rl(stats=None) == -6
    assert rl(N=736, ldr=736, ldx=736, ldy=736) == -2                               # N % 64
    assert rl(Y=A16 + 4) == -4 and rl(ldy=766) == -4                                # Y layout
    assert rl(sw=10) == -2 and rl(syw=2) == -2                                      # statistics / sync words
    rr = lambda **kw: lib.mx_gemm_bf16_res_rms(*{**dict(
        st=None, A=A16, lda=768, W=A16, ldw=768, bias=A16, R=A16, ldr=768, X=A16, ldx=768, sc1=A16, Y=A16, ldy=768,
        M=1280, N=768, K=768, Kw=768, eps=1e-6, stats=A16, sw=1 << 20, sync=A16, syw=1 << 10), **kw}.values())
    assert rr(sc1=None) == -6 and rr(X=None) == -6 and rr(sync=None) == -6
    assert rr(N=736, ldr=736, ldx=736, ldy=736) == -2
    assert rr(sc1=A16 + 2) == -4 and rr(stats=A16 + 8) == -4
    assert rr(sw=10) == -2
    assert lib.mx_gemm_res_ln_stats_words(1280, 768) == 20 * 12 * 64 * 2 and lib.mx_gemm_res_ln_sync_words(1280) == 21
    # tracking heads
    assert lib.mx_track_head_blob_elems(768, 256, 512) == 768 * 256 + 6 * 256 + 256 * 256 + 256 * 512 + 512
    hd = lambda **kw: lib.mx_track_heads(*(lambda a: (a.update(kw), list(a.values()))[1])(dict(
        st=None, x=A16, ldx=768, Q=256, D=768, H=256, cb=A16, NOC=512, ce0=1e-5, ce1=1e-5, vb=A16, ve0=1e-5,
        ve1=1e-5, radius=20, tr=A16, lg=A16, ldl=512, vis=A16)))
    assert hd(H=257) == -2             # more hidden units than threads
    assert hd(NOC=511) == -2           # odd coordinate logits
    assert hd(NOC=1026, ldl=1026) == -2  # 513 bins per half
    assert hd(ldl=500) == -2
    assert hd(radius=-1) == -2
    assert hd(vb=None) == -6
    assert hd(Q=0, x=None) == 0        # nothing to do
    # W8A8
    assert lib.mx_quant_rows_i8(None, A16, 2048, A16, 2048, A16, 4, 2044) == -2                 # K % 8
    assert lib.mx_quant_rows_i8(None, A16 + 8, 2048, A16, 2048, A16, 4, 2048) == -4             # x not 16-byte aligned
    assert lib.mx_quant_rows_i8(None, A16, 2048, None, 2048, A16, 4, 2048) == -6
    assert lib.mx_quant_weight_i8(None, A16, 2048, A16, 2040, A16, 4, 2048) == -2            # ldq < K
    i8 = lambda **kw: lib.mx_gemm_i8(*{**dict(st=None, cfg=0, A=A16, lda=2048, W=A16, ldw=2048, sa=A16, sw=A16,
                                                bias=A16, R=None, ldr=0, r_rows=0, C=A16, ldc=2048, M=64, N=2048,
                                                K=2048, Kw=2048, act=0, P=None, ldp=0), **kw}.values())
    assert i8(K=2040, lda=2040) == -2 and i8(Kw=2000) == -2 and i8(lda=2056 - 4) == -2
    assert i8(cfg=8) == -1                                                          # wave-split configs: bf16 only
    assert i8(cfg=15, P=A16, ldp=2048) == -1                                        # raw int32 needs a partial-sum cfg
    assert i8(act=3) == -1 and i8(A=A16 + 8) == -4 and i8(sw=None) == -6


def test_generate_refuses_to_overrun_the_kv_cache():
    """A prefill of 1 + 729 + 64 tokens leaves 1024 - 794 = 230 decode steps in a 1024-entry cache: generate() of
    231 tokens fits, of 232 raises ValueError before any device work (the check needs no GPU)."""
    import strix_halo_maxx_amd.md2text as mt
    dec = mt.TextDecoder.__new__(mt.TextDecoder)
    dec.ctx = 1024
    img, prompt = torch.zeros(729, 2048), torch.zeros(64, dtype=torch.long)
    dec._check_room(1 + 729 + 64, 231)
    with pytest.raises(ValueError):
        dec.generate(img, prompt, 232)
    with pytest.raises(ValueError):
        dec._check_room(1024, 2)
    dec.pos_base, dec.steps = 1000, 24
    with pytest.raises(ValueError):
        dec._count_step()
