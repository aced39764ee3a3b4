"""GPU parity: every row configuration of the log-sum-exp row engine, with
enough rows that each workgroup of the persistent grid walks several of them.

The row kernels (CrossEntropy train and inference, selective log-softmax,
GRPO with and without the gradient) pick a configuration from the row length:
register-resident rows on 256, 512 or 1024 lanes with 1 to 24 16-byte vectors
a lane, or a streaming loop. The grid holds as many workgroups as the CUs
keep resident (256 x occupancy, at most 2048), and a workgroup walks rows
blockIdx, blockIdx + grid, ... with the next row's loads overlapping the
current row's reduction. These tests size the row count above the largest
grid so that the later rows of a workgroup (the refilled registers) are
checked against the oracle, not only the first one.
"""
import math

import pytest
import torch

import oracle
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_cross_entropy, hilda_grpo_loss, fused_selective_log_softmax

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32

# (V, dtype) -> the configuration it selects (16-byte vectors: 8 bf16 or 4 fp32 elements)
CE_CONFIGS = [
    (1000, BF16),     # 256 lanes x 1
    (4000, BF16),     # 256 x 2
    (8000, BF16),     # 256 x 4
    (12000, BF16),    # 256 x 8
    (20000, BF16),    # 256 x 12
    (32000, BF16),    # 512 x 8
    (45000, BF16),    # 512 x 12
    (60000, BF16),    # 512 x 16
    (90000, BF16),    # 1024 x 12
    (128256, BF16),   # 1024 x 16
    (151936, BF16),   # 1024 x 20
    (180000, BF16),   # 1024 x 24
    (200000, BF16),   # streaming
    (20000, F32),     # 512 x 12
    (60000, F32),     # 1024 x 16
    (90000, F32),     # 1024 x 24
]


def _rows_for(V, dtype):
    # past the largest grid of the row's configuration (2048 workgroups of 256 lanes)
    nv = V * torch.tensor([], dtype=dtype).element_size() // 16
    return 2200 if nv <= 4096 else 600


@pytest.mark.parametrize("V,dtype", CE_CONFIGS)
def test_cross_entropy_row_configs(V, dtype):
    dev = gpu()
    N = _rows_for(V, dtype)
    g = torch.Generator(device=dev).manual_seed(V)
    logits = (2 * torch.randn(N, V, generator=g, device=dev)).to(dtype)
    t = torch.randint(0, V, (N,), generator=g, device=dev)
    t[torch.rand(N, generator=g, device=dev) < 0.2] = -100
    print(f"CE V={V} {dtype} rows={N}", flush=True)
    lg = logits.clone().requires_grad_(True)
    train = hilda_cross_entropy(lg, t, -100, "none")  # fused loss + gradient kernel
    train.backward(torch.ones(N, device=dev))
    with torch.no_grad():
        infer = hilda_cross_entropy(logits, t, -100, "none")  # inference (lse) kernel
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == F32 else dict(rtol=2e-3, atol=2e-3)
    # the first rows and the last ones (the last rows of their workgroups)
    rows = torch.cat([torch.arange(8), torch.arange(N - 40, N)])
    sub = logits[rows.to(dev)].cpu()
    ts = t[rows.to(dev)].cpu()
    (l_ref,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, ts, -100, "none"), [sub],
                                        [torch.ones(len(rows))], dtype=torch.float64)
    assert_close(train[rows.to(dev)], l_ref, name="train loss rows", **lt)
    assert_close(infer[rows.to(dev)], l_ref, name="inference loss rows", **lt)
    assert_close(lg.grad[rows.to(dev)], d_ref, name="dlogits rows", **tol(dtype))
    assert rel_fro(lg.grad[rows.to(dev)], d_ref.to(dtype)) < (1e-5 if dtype == F32 else 1e-2)
    # every row: both kernels agree, gradient rows of live targets sum to ~0, ignored rows are zero
    assert_close(infer, train, name="inference vs train (all rows)", **lt)
    ign = t == -100
    assert torch.count_nonzero(lg.grad[ign]).item() == 0
    assert torch.count_nonzero(train[ign]).item() == 0
    row_sums = lg.grad[~ign].float().sum(-1)
    assert row_sums.abs().max().item() < (1e-4 if dtype == F32 else 2e-2)


GRPO_CONFIGS = [
    (8000, BF16),     # 256 x 4
    (20000, BF16),    # 256 x 12
    (32000, BF16),    # 512 x 8
    (45000, BF16),    # 512 x 12
    (60000, BF16),    # 512 x 16
    (90000, BF16),    # 1024 x 12
    (151936, BF16),   # 1024 x 20
    (180000, BF16),   # 1024 x 24
    (200000, BF16),   # streaming
    (20000, F32),     # 512 x 12
]


@pytest.mark.parametrize("V,dtype", GRPO_CONFIGS)
def test_grpo_row_configs(V, dtype):
    """GRPO with and without the gradient and the selective log-softmax over
    several rows a workgroup; two sequences checked against the oracle run on
    them alone (the per-sequence terms do not depend on the other sequences
    except through the 1/B factor)."""
    dev = gpu()
    rows = _rows_for(V, dtype)
    B = 3 if rows > 1000 else 4
    L = rows // B
    g = torch.Generator(device=dev).manual_seed(V + 1)
    logits = (2 * torch.randn(B, L + 1, V, generator=g, device=dev)).to(dtype)
    ids = torch.randint(0, V, (B, L), generator=g, device=dev)
    adv = torch.randn(B, generator=g, device=dev)
    old = -math.log(V) + 0.5 * torch.randn(B, L, generator=g, device=dev)
    ref = -math.log(V) + 0.5 * torch.randn(B, L, generator=g, device=dev)
    lens = torch.tensor([L, L // 2, (3 * L) // 4, L - 3][:B], device=dev)
    mask = (torch.arange(L, device=dev)[None, :] < lens[:, None]).to(torch.int32)
    args = (ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    print(f"GRPO V={V} {dtype} B={B} L={L}", flush=True)
    lg = logits.clone().requires_grad_(True)
    loss, kl, clip = hilda_grpo_loss(lg, *args)
    loss.backward()
    with torch.no_grad():
        l_ng, kl_ng, clip_ng = hilda_grpo_loss(logits, *args)
    # the forward-only kernel reduces exactly as the gradient kernel does
    assert torch.equal(l_ng, loss.detach()) and torch.equal(kl_ng, kl) and torch.equal(clip_ng, clip)
    grad = lg.grad
    assert torch.count_nonzero(grad[:, -1]).item() == 0
    assert torch.count_nonzero(grad[:, :-1][mask == 0]).item() == 0
    full_ids = torch.cat([torch.zeros_like(ids[:, :1]), ids], 1)
    full_mask = torch.cat([torch.ones_like(mask[:, :1]), mask], 1)
    logp = fused_selective_log_softmax(logits, full_ids, 1.0, full_mask)
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == F32 else dict(rtol=1e-4, atol=1e-4)
    per_seq = []
    for b in range(B):
        checked = b in (0, B - 1)
        dt = torch.float64 if checked else torch.float32
        lb = logits[b:b + 1].cpu().to(dt).requires_grad_(checked)
        sargs = (ids[b:b + 1].cpu(), adv[b:b + 1].cpu().to(dt), old[b:b + 1].cpu().to(dt),
                 ref[b:b + 1].cpu().to(dt), mask[b:b + 1].cpu(), 1.0, 0.1, 0.2, 0.2)
        lo, _, _ = oracle.grpo_loss_ref(lb, *sargs)
        per_seq.append(lo.item())
        if checked:
            lo.backward()
            d = lb.grad[0] / B  # the oracle saw batch size 1
            s = B * float(mask[b].sum())
            assert_close(grad[b].float() * s, d * s, name=f"seq {b} grad", **tol(dtype))
            lp_ref = oracle.selective_log_softmax_ref(lb.detach(), full_ids[b:b + 1].cpu(), 1.0,
                                                      full_mask[b:b + 1].cpu())
            assert_close(logp[b:b + 1], lp_ref, name=f"seq {b} logp", **lt)
    assert math.isclose(loss.item(), sum(per_seq) / B, rel_tol=2e-3, abs_tol=2e-3)
