"""GPU: llmt_cross_entropy_noalloc (the allocation-free variant of
llmt_cross_entropy, its statistics in the library's built-in device scratch)
against llmt_cross_entropy through the C ABI, bit for bit, on two calls in a
row with the second one smaller, and the host-side rejection of inputs larger
than the scratch."""
import ctypes as C

import pytest
import torch

import llmt

pytestmark = pytest.mark.gpu

vp, i32 = C.c_void_p, C.c_int


def _fn():
    f = llmt.lib().llmt_cross_entropy_noalloc
    f.restype = i32
    f.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp]
    return f


def _run(fn, logits, tgt, seq_len, dev):
    rows, V = logits.shape
    dl = torch.full((rows, V), float("nan"), device=dev)
    lr = torch.full((rows,), float("nan"), device=dev)
    lm = torch.full((1,), float("nan"), device=dev)
    torch.cuda.synchronize()
    rc = fn(logits.data_ptr(), tgt.data_ptr(), rows, V, seq_len, dl.data_ptr(), lr.data_ptr(),
            lm.data_ptr(), None)
    assert rc == llmt.LLMT_OK, llmt.lib().llmt_last_error().decode()
    torch.cuda.synchronize()
    return dl, lr, lm


@pytest.mark.parametrize("first,second", [((256, 151936, 128), (64, 50000, 32))])
def test_noalloc_cross_entropy_matches_allocating(dev, first, second):
    L = llmt.lib()
    noalloc = _fn()
    alloc = L.llmt_cross_entropy
    g = torch.Generator(device=dev).manual_seed(11)
    for rows, V, S in (first, second):
        print(f"case: cross_entropy_noalloc rows {rows} V {V} S {S}", flush=True)
        logits = torch.randn(rows, V, generator=g, device=dev) * 3.0
        tgt = torch.randint(0, V, (rows,), generator=g, device=dev, dtype=torch.int32)
        got = _run(noalloc, logits, tgt, S, dev)
        want = _run(alloc, logits, tgt, S, dev)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_noalloc_rejects_inputs_beyond_the_scratch(dev):
    noalloc = _fn()
    V = 151936
    rows = 14000   # 14000 x 19 chunks > the 262144 statistics of the scratch
    rc = noalloc(vp(256), vp(256), rows, V, 2, None, vp(256), None, None)
    assert rc == llmt.LLMT_ERR_ARG
    assert "exceed" in llmt.lib().llmt_last_error().decode()
