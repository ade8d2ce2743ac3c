"""GPU parity of the standalone operators (through the C ABI) against the
oracle / a plain fp32 reference of the same op."""
import numpy as np
import pytest
import torch

import llmt
from helpers import rel_l2
from oracle import lora_step as ref
from oracle.quant import quantize_rows

pytestmark = pytest.mark.gpu


def _seed(s):
    return torch.Generator().manual_seed(s)


# M >= 1024 (a multiple of 256) takes the 256 x 128 tile kernel, including
# partial last column tiles (2064, 4144 = 4096 + 48).
@pytest.mark.parametrize("M,N,K", [(16, 64, 64), (32, 2064, 2048), (128, 4096 + 48, 2048),
                                   (128, 2048, 6144), (64, 12288, 2048), (256, 1024, 2048),
                                   (128, 2048, 12288), (48, 160, 320), (1024, 2064, 2048),
                                   (2048, 4096 + 48, 512), (1024, 384, 4096)])
def test_gemm_f16_matches_fp32(dev, L, M, N, K):
    g = _seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g).half()
    B = (torch.randn(N, K, generator=g) * 0.02).half()
    want = A.float() @ B.float().t()
    got = llmt.gemm_f16(A.to(dev), B.to(dev)).cpu()
    assert rel_l2(got, want) < 1e-5
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("nb,stages", [("2", "4"), ("3", "3"), ("4", "4"), ("6", "3"), ("8", "4"),
                                       ("4", "0"), ("3", "5"), ("8", "5"), ("4", "6"),
                                       ("3", "6")])
@pytest.mark.parametrize("M,N,K", [(128, 2048 + 48, 2048), (256, 160, 4096), (128, 12288, 1024),
                                   (128, 512, 64), (128, 256, 192), (128, 4096, 320)])
def test_gemm_f16_skinny_tiles(dev, L, monkeypatch, nb, stages, M, N, K):
    """Every tile width (nb 16-column fragments) / ring depth of the
    M % 128 == 0 path (0 stages: the register-staged kernel), including
    partial last column tiles and reductions shorter than the ring
    (K / 64 = 1, 3, 5 stages)."""
    monkeypatch.setenv("LLMT_GEMM_SKINNY_NB", nb)
    monkeypatch.setenv("LLMT_GEMM_SKINNY_STAGES", stages)
    g = _seed(M + N + K + int(nb))
    A = torch.randn(M, K, generator=g).half()
    B = (torch.randn(N, K, generator=g) * 0.02).half()
    want = A.float() @ B.float().t()
    got = llmt.gemm_f16(A.to(dev), B.to(dev)).cpu()
    assert rel_l2(got, want) < 1e-5
    assert torch.isfinite(got).all()


def test_gemm_f16_lm_head_dx_shape(dev, L):
    # dX of the lm_head: reduction over the full vocabulary (K = 151936).
    g = _seed(11)
    M, N, K = 128, 256, 151936
    A = (torch.randn(M, K, generator=g)).half()
    B = (torch.randn(N, K, generator=g) * 0.02).half()
    want = A.float() @ B.float().t()
    got = llmt.gemm_f16(A.to(dev), B.to(dev)).cpu()
    assert rel_l2(got, want) < 1e-5


def test_gemm_strided_operands(dev, L):
    g = _seed(12)
    A = torch.randn(32, 256, generator=g).half()
    B = (torch.randn(48, 192, generator=g)).half()
    Ad, Bd = A.to(dev), B.to(dev)
    out = torch.full((32, 80), -7.0, device=dev)
    llmt.gemm_f16(Ad[:, :128], Bd[:, :128], out=out[:, :48])
    want = A[:, :128].float() @ B[:, :128].float().t()
    assert rel_l2(out[:, :48].cpu(), want) < 1e-5
    assert (out[:, 48:] == -7.0).all()


@pytest.mark.parametrize("M", [128, 1024])
def test_gemm_i8_matches_dequant(dev, L, M):
    g = _seed(13)
    N, K = 1024, 2048
    A = torch.randn(M, K, generator=g).half()
    w = torch.randn(N, K, generator=g) * 0.02
    q, sc = quantize_rows(w.numpy())
    sc16 = torch.from_numpy(sc.astype(np.float16))
    qt = torch.from_numpy(q)
    want = (A.float() @ qt.float().t()) * sc16.float()[None, :]
    got = llmt.gemm_i8(A.to(dev), qt.to(dev), sc16.to(dev)).cpu()
    assert rel_l2(got, want) < 1e-5


def test_quantize_bit_exact(dev, L):
    g = _seed(14)
    w = torch.randn(257, 2048, generator=g) * 0.02
    # ties: w*inv lands exactly on k + 0.5 -> round half to even
    w[0, :6] = torch.tensor([127.0, 0.5, 1.5, -2.5, 2.5, -0.5])
    w[1] = 0.0                     # all-zero row: scale 0, inv 0, q 0
    w[2, :3] = torch.tensor([1e-30, -3e-38, 0.0])
    q_ref, s_ref = quantize_rows(w.numpy())
    q, s = llmt.quantize_rows_i8(w.to(dev))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("rows,V,seq_len", [(128, 151936, 128), (64, 151936, 16), (32, 512, 8)])
def test_cross_entropy_matches_oracle(dev, L, rows, V, seq_len):
    g = _seed(rows + V)
    logits = torch.randn(rows, V, generator=g) * 2.0
    targets = torch.randint(0, V, (rows,), generator=g, dtype=torch.int32)
    valid = ref.valid_rows(rows // seq_len, seq_len)
    loss_ref, dl_ref, rows_ref = ref.cross_entropy(logits, targets, valid)
    lm, lr, dl = llmt.cross_entropy(logits.to(dev), targets.to(dev), seq_len)
    assert abs(float(lm) - float(loss_ref)) < 1e-3          # loss: 1e-3 absolute
    assert rel_l2(lr.cpu()[valid], rows_ref[valid]) < 1e-5
    assert (lr.cpu()[~valid] == 0).all()
    dl = dl.cpu()
    assert rel_l2(dl, dl_ref) < 1e-2                          # grads: 1e-2 rel L2
    assert rel_l2(dl, dl_ref) < 1e-4                          # (actual headroom)
    assert (dl[~valid] == 0).all()                            # Q4: zero rows
    # each valid row of dlogits sums to ~0 (softmax minus one-hot)
    assert dl[valid].double().sum(-1).abs().max() < 1e-6


def test_cross_entropy_known_answer(dev, L):
    # all-zero logits: loss = ln V exactly, dlogits = (1/V - 1[t]) / n_valid
    V, S = 151936, 16
    logits = torch.zeros(S, V, device=dev)
    targets = torch.arange(S, dtype=torch.int32, device=dev) * 7
    lm, lr, dl = llmt.cross_entropy(logits, targets, S)
    assert abs(float(lm) - np.log(V)) < 1e-4
    assert abs(float(dl[0, 1]) - (1.0 / V) / (S - 1)) < 1e-9
    assert abs(float(dl[0, 0]) - (1.0 / V - 1.0) / (S - 1)) < 1e-7
