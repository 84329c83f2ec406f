"""tsfm_qkv_project_noalloc: the projection entry point that allocates nothing (its split partial
sums live in a fixed device array of the library), against tsfm_qkv_project on the same inputs,
through the C ABI. Bit-identical outputs are required: both run the same kernels with the same
split of the reduction (16 tokens or fewer: the 16-token kernel, no partials in the array). Two
calls in a row (the second smaller) reuse the array; the largest partials the split rule can
produce fit it; host pointers are refused before anything is queued.
"""
import ctypes

import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu


def _lib(ta):
    return ta.load()


def _case(torch, seed, tokens, d, nh, gated=False, rope=False):
    rng = np.random.default_rng(seed)
    inner = nh * 64
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x = cu(rng.standard_normal((tokens, d)).astype(np.float32))
    n_w = 4 if gated else 3
    ws = [cu((rng.standard_normal((inner, d)) / np.sqrt(d)).astype(np.float32)) for _ in range(n_w)]
    tabs = None
    if rope:
        c, s = _ref.timestral_rope_tables(1, tokens, tokens, 0, 64, 64, 10000.0, [0])
        tabs = (cu(c), cu(s))
    return x, ws, tabs, tokens, d, nh


def _args(ta, c, outs):
    x, ws, tabs, tokens, d, nh = c
    inner = nh * 64
    gated = len(ws) == 4
    return ta.ProjArgs(dtype=ta.DTYPE_F32, out_dtype=ta.DTYPE_F32, batch=1, seq=tokens, d_in=d, heads=nh, head_dim=64,
                       flags=ta.DEVICE_PTRS, rope_half=32 if tabs else 0, rope_rows_per_table=0, rope_row0=0,
                       rope_table_stride=0, x=x.data_ptr(), x_tok=d, w_q=ws[0].data_ptr(), w_k=ws[1].data_ptr(),
                       w_v=ws[2].data_ptr(), w_gate=ws[3].data_ptr() if gated else None,
                       q=outs[0].data_ptr(), q_tok=inner, k=outs[1].data_ptr(), k_tok=inner, v=outs[2].data_ptr(),
                       v_tok=inner, gate=outs[3].data_ptr() if gated else None, gate_tok=inner if gated else 0,
                       rope_cos=tabs[0].data_ptr() if tabs else None, rope_sin=tabs[1].data_ptr() if tabs else None,
                       stream=0)


def _run(torch, ta, fn, c):
    x, ws, tabs, tokens, d, nh = c
    outs = [torch.full((tokens, nh * 64), -7.0, dtype=torch.float32, device="cuda") for _ in ws]
    rc = fn(ctypes.byref(_args(ta, c, outs)))
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("first,second", [((300, 256, 4, True), (48, 256, 4, False)),
                                          ((528, 512, 8, False), (16, 512, 8, True))])
def test_noalloc_matches_the_allocating_entry_point(ta, gpu_ready, first, second):
    """Split products (their partials in the fixed array), a gated four-output product, and a
    second, smaller call right after the first: every output has the bits of tsfm_qkv_project."""
    import torch

    lib = _lib(ta)
    for i, (tokens, d, nh, gated) in enumerate((first, second)):
        c = _case(torch, 10 + i + tokens, tokens, d, nh, gated=gated)
        want = _run(torch, ta, lib.tsfm_qkv_project, c)
        got = _run(torch, ta, lib.tsfm_qkv_project_noalloc, c)
        for g, w_ in zip(got, want):
            assert np.array_equal(g, w_)


def test_noalloc_unsplit_with_rope(ta, gpu_ready):
    """A product large enough to run unsplit (no partials), with RoPE in the epilogue."""
    import torch

    lib = _lib(ta)
    c = _case(torch, 5, 4096, 256, 4, rope=True)
    want = _run(torch, ta, lib.tsfm_qkv_project, c)
    got = _run(torch, ta, lib.tsfm_qkv_project_noalloc, c)
    for g, w_ in zip(got, want):
        assert np.array_equal(g, w_)


def test_noalloc_refuses_host_pointers(ta, gpu_ready):
    lib = _lib(ta)
    # Host pointers: refused (the call would have to stage them in allocated memory).
    x = np.zeros((16, 64), np.float32)
    w = np.zeros((64, 64), np.float32)
    y = [np.zeros((16, 64), np.float32) for _ in range(3)]
    a = ta.ProjArgs(dtype=ta.DTYPE_F32, out_dtype=ta.DTYPE_F32, batch=1, seq=16, d_in=64, heads=1, head_dim=64, flags=0,
                    x=x.ctypes.data, x_tok=64, w_q=w.ctypes.data, w_k=w.ctypes.data, w_v=w.ctypes.data,
                    q=y[0].ctypes.data, q_tok=64, k=y[1].ctypes.data, k_tok=64, v=y[2].ctypes.data, v_tok=64)
    assert lib.tsfm_qkv_project_noalloc(ctypes.byref(a)) == ta.E_UNSUPPORTED


def test_noalloc_holds_the_largest_split_partials(ta, gpu_ready):
    """The split rule aims at about 512 workgroups: a product of b < 512 tiles of 64 x 64 splits
    ceil(512 / b) ways at most, so its partials never exceed 2 x 511 tiles (16.7 MB, under the
    array's 16 MiB). 448 tokens x 3 x 24 heads = 7 x 72 = 504 tiles, two splits over d_in 256:
    16.5 MB of partials, the same bits as tsfm_qkv_project."""
    import torch

    lib = _lib(ta)
    c = _case(torch, 6, 448, 256, 24)
    want = _run(torch, ta, lib.tsfm_qkv_project, c)
    got = _run(torch, ta, lib.tsfm_qkv_project_noalloc, c)
    for g, w_ in zip(got, want):
        assert np.array_equal(g, w_)
