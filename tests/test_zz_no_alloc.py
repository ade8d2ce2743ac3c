"""GPU: llmt_cross_entropy_noalloc (the allocation-free variant of
llmt_cross_entropy, its statistics in the library's built-in device scratch)
against llmt_cross_entropy through the C ABI, bit for bit, on two calls in a
row with the second one smaller, and as the first call of a process captured
into a graph and replayed.  (The host-side rejection of inputs larger than the
scratch is a CPU test, tests/test_library.py.)"""
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


_CAPTURE_SCRIPT = r"""
import sys
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/llm.cu_amd"]
import ctypes as C
import torch
import llmt
vp, i32 = C.c_void_p, C.c_int
L = llmt.lib()
f = L.llmt_cross_entropy_noalloc
f.restype = i32
f.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp]
dev = torch.device("cuda:0")
rows, V, S = 128, 151936, 64
g = torch.Generator(device=dev).manual_seed(5)
logits = torch.randn(rows, V, generator=g, device=dev) * 3.0
tgt = torch.randint(0, V, (rows,), generator=g, device=dev, dtype=torch.int32)
dl = torch.empty(rows, V, device=dev)
lr = torch.empty(rows, device=dev)
lm = torch.empty(1, device=dev)
torch.cuda.synchronize()
print("case: first noalloc call of the process, under graph capture", flush=True)
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        rc = f(logits.data_ptr(), tgt.data_ptr(), rows, V, S, dl.data_ptr(), lr.data_ptr(),
               lm.data_ptr(), torch.cuda.current_stream().cuda_stream)
assert rc == 0, L.llmt_last_error().decode()
for rep in range(3):
    logits.mul_(1.25).add_(0.5)
    tgt.copy_(torch.randint(0, V, (rows,), generator=g, device=dev, dtype=torch.int32))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    want = [torch.full_like(t, float("nan")) for t in (dl, lr, lm)]
    assert L.llmt_cross_entropy(vp(logits.data_ptr()), vp(tgt.data_ptr()), rows, V, S,
                                vp(want[0].data_ptr()), vp(want[1].data_ptr()),
                                vp(want[2].data_ptr()), None) == 0
    torch.cuda.synchronize()
    for a, b in zip((dl, lr, lm), want):
        assert torch.equal(a, b), rep
    print(f"replay {rep} bit-exact", flush=True)
print("ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(dev):
    """A caller that captures llmt_cross_entropy_noalloc into a graph before
    any other call of it in the process (the scratch address is then looked
    up inside the capture): three replays, each after new logits and targets
    were written in place, equal the allocating call bit for bit.  Runs in a
    fresh process so that the captured call is the first one."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_SCRIPT, str(root)],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.rstrip().endswith("ok")
