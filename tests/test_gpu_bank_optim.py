"""The bank optimizer on the GPU (BankAdamW, RowSparseBankGrad, clip_grad_norm_) against the
oracle's AdamW and clip_grad_norm (torch.optim.AdamW and torch.nn.utils.clip_grad_norm_ as the
reference runs them, training/trainer.py:309-392, :876-889), in float64 on the CPU.

fp32 tolerance: 1e-5 relative max error (max |a - b| / max |b|) on parameters and moments.
Row-sparse runs are compared with the oracle's *dense* steps (zero gradient rows included), at
every read of a chapter (after the layer-side catch-up) and after a final flush."""

import copy

import pytest
import torch

import oracle as O
from helpers import assert_rel, gen

pytestmark = pytest.mark.gpu

BETAS, EPS, WD = (0.9, 0.95), 1e-8, 0.1


def _lr(step):
    return 6e-3 * min(1.0, step / 3.0) * (1.0 - 0.05 * step)   # warm-up, then decay


@pytest.fixture(scope="module")
def dev(gpu_device):
    from memory_amd import _lib
    _lib.lib()
    return gpu_device


def _rows(chapters, T):
    return (chapters[:, None] * T + torch.arange(T)[None, :]).reshape(-1)


@pytest.mark.parametrize("C,T,d", [(9, 4, 24), (5, 8, 392), (3, 64, 768)])
def test_dense_steps_match_oracle(dev, C, T, d):
    print(f"bank adamw dense C={C} T={T} d={d}", flush=True)
    from memory_amd.bank_optim import BankAdamW
    g0 = gen(C * T + d)
    p0 = torch.randn(C * T, d, generator=g0)
    bank = torch.nn.Parameter(p0.clone().to(dev))
    opt = BankAdamW(bank, T, lr=_lr(1), betas=BETAS, eps=EPS, weight_decay=WD, row_sparse=False,
                    mirror_dtype=torch.bfloat16)
    p, m, v = p0.double(), torch.zeros(C * T, d, dtype=torch.float64), torch.zeros(C * T, d, dtype=torch.float64)
    for step in range(1, 6):
        lr = _lr(step)
        opt.param_groups[0]["lr"] = lr
        g = torch.randn(C * T, d, generator=g0)
        bank.grad = g.to(dev)
        opt.step()
        opt.zero_grad()
        O.adamw_step(p, g.double(), m, v, step, lr, BETAS, EPS, WD)
    assert_rel(bank.detach(), p, 1e-5, "param")
    assert_rel(opt.exp_avg, m, 1e-5, "exp_avg")
    assert_rel(opt.exp_avg_sq, v, 1e-5, "exp_avg_sq")
    assert torch.equal(opt.mirror.cpu(), bank.detach().cpu().to(torch.bfloat16))


@pytest.mark.parametrize("C,T,d,steps", [(12, 4, 40, 10), (6, 16, 256, 7), (4, 64, 96, 300)])
def test_row_sparse_lazy_steps_match_dense_oracle(dev, C, T, d, steps):
    """Random chapters touched per step; chapter C-1 never, chapter C-2 only in the last step
    (its whole history replayed at once; with 300 steps the replay crosses the 256-step staging
    of the scalar history); gradient clipping on odd steps."""
    print(f"bank adamw row-sparse C={C} T={T} d={d} steps={steps}", flush=True)
    from memory_amd.bank_optim import BankAdamW, clip_grad_norm_
    g0 = gen(7 * C + d + steps)
    p0 = torch.randn(C * T, d, generator=g0)
    bank = torch.nn.Parameter(p0.clone().to(dev))
    opt = BankAdamW(bank, T, lr=_lr(1), betas=BETAS, eps=EPS, weight_decay=WD, mirror_dtype=torch.bfloat16)
    p, m, v = p0.double(), torch.zeros(C * T, d, dtype=torch.float64), torch.zeros(C * T, d, dtype=torch.float64)
    for step in range(1, steps + 1):
        lr = _lr(step) if steps <= 20 else 6e-3 * (1.0 - 0.002 * step)
        opt.param_groups[0]["lr"] = lr
        pool = torch.randperm(C - 2, generator=g0)
        ch = pool[: max(1, (C - 2) // 2)].sort().values
        if step == steps:
            ch = torch.cat([ch, torch.tensor([C - 2])])
        # the "forward": the layer brings its chapters to the last step, then reads them
        chd = ch.to(dev, torch.int32)
        opt.catch_up(chd, torch.tensor([ch.numel()], device=dev, dtype=torch.int32), ch.numel())
        rows = _rows(ch, T)
        assert_rel(bank.detach()[rows.to(dev)], p[rows], 1e-5, f"rows read at step {step}")
        assert_rel(opt.mirror[rows.to(dev)].float(), p[rows].float().to(torch.bfloat16).float(), 1e-2,
                   f"mirror rows at step {step}")
        grows = torch.randn(ch.numel() * T, d, generator=g0)
        opt.row_grad.add_(chd, grows.to(dev))
        g = torch.zeros(C * T, d, dtype=torch.float64)
        g[rows] = grows.double()
        if step % 2 == 1:
            total = clip_grad_norm_([bank], 0.5)
            total_ref = O.clip_grad_norm([g], 0.5)
            assert abs(float(total) - float(total_ref)) <= 1e-5 * float(total_ref)
        opt.step()
        opt.zero_grad()
        O.adamw_step(p, g, m, v, step, lr, BETAS, EPS, WD)
    opt.flush()
    assert_rel(bank.detach(), p, 1e-5, "param after flush")
    assert_rel(opt.exp_avg, m, 1e-5, "exp_avg")
    assert_rel(opt.exp_avg_sq, v, 1e-5, "exp_avg_sq")
    assert torch.equal(opt.mirror.cpu(), bank.detach().cpu().to(torch.bfloat16))


def test_sparse_grad_norm_and_dense_view(dev):
    from memory_amd.bank_optim import RowSparseBankGrad
    C, T, d = 10, 8, 64
    g0 = gen(31)
    bank = torch.nn.Parameter(torch.randn(C * T, d, generator=g0).to(dev))
    rg = RowSparseBankGrad(bank, T)
    dense = torch.zeros(C * T, d, dtype=torch.float64)
    for chs in ([3, 7, 1], [7, 2], [9]):          # chapter 7 twice: the second contribution adds
        ch = torch.tensor(chs)
        rows = torch.randn(len(chs) * T, d, generator=g0)
        rg.add_(ch, rows.to(dev))
        dense[_rows(ch, T)] += rows.double()
    lst, n = rg.touched()
    assert lst[: int(n.item())].cpu().tolist() == [1, 2, 3, 7, 9]
    assert_rel(rg.to_dense(), dense, 1e-6, "dense view")
    assert abs(float(rg.sqnorm()) - float((dense ** 2).sum())) <= 1e-5 * float((dense ** 2).sum())
    rg.zero_()
    assert not rg.has_rows and float(rg.sqnorm()) == 0.0
    rg.add_(torch.tensor([7]), torch.ones(T, d).to(dev))    # a new epoch stores, it does not add
    assert_rel(rg.to_dense()[7 * T:8 * T], torch.ones(T, d), 0.0, "fresh epoch")


def _layer(D, H, C, T, K, seed, normalize=False):
    from memory_amd.model import RoutedMemoryLayer
    torch.manual_seed(seed)
    return RoutedMemoryLayer(D, H, C, T, K, num_shared_chapters=1, routed_scaling_factor=2.5,
                             normalize_shared_routed_before_mixing=normalize, wo_init_zero=False)


@pytest.mark.parametrize("dtype,normalize", [(torch.bfloat16, False), (torch.float32, True)])
def test_layer_row_sparse_grad_equals_dense(dev, dtype, normalize):
    """Two memory layers sharing one fp32 bank, two micro-batches: the rows accumulated by the
    layers' backward equal the dense autograd gradient of the bank."""
    print(f"layer row-sparse bank grad {dtype} normalize={normalize}", flush=True)
    from memory_amd.bank_optim import RowSparseBankGrad
    D, H, C, T, K = 128, 2, 17, 64, 4
    layers = [_layer(D, H, C, T, K, s, normalize).to(dev) for s in (1, 2)]
    for lay in layers:
        for mod in (lay.memory_attn.q_proj, lay.memory_attn.k_proj, lay.memory_attn.v_proj, lay.memory_attn.o_proj):
            mod.to(dtype)
    g0 = gen(41)
    bank = torch.nn.Parameter((torch.randn(C * T, D, generator=g0) * 0.5).to(dev))
    hs = [torch.randn(2, 96, D, generator=g0).to(dev, dtype) for _ in range(2)]

    def run():
        for h in hs:
            x = h
            for lay in layers:
                y, _ = lay(x, bank, return_losses=False)
                x = x + y
            (x.float() ** 2).mean().backward()

    run()
    dense = bank.grad.detach().clone()
    bank.grad = None
    rg = RowSparseBankGrad(bank, T)
    run()
    assert bank.grad is None
    assert_rel(rg.to_dense(), dense, 1e-5, "row-sparse bank grad")


def test_training_steps_match_torch_adamw(dev):
    """Four training steps of a sequence memory layer: BankAdamW (row-sparse, lazy catch-up)
    against torch.optim.AdamW on the dense bank gradient, both after clip_grad_norm_ over the
    bank and the layer's parameters.  The layer outputs of every step (which read the caught-up
    chapters) and the final bank agree."""
    print("training steps: BankAdamW vs torch AdamW", flush=True)
    from memory_amd.bank_optim import BankAdamW, clip_grad_norm_
    D, H, C, T, K = 128, 2, 33, 64, 4
    g0 = gen(51)
    bank0 = torch.randn(C * T, D, generator=g0) * 0.5
    hs = [torch.randn(2, 80, D, generator=g0).to(dev) for _ in range(4)]
    outs = {}
    for kind in ("torch", "bank_adamw"):
        layer = _layer(D, H, C, T, K, 3).to(dev)
        bank = torch.nn.Parameter(bank0.clone().to(dev))
        if kind == "torch":
            opt = torch.optim.AdamW([bank], lr=_lr(1), betas=BETAS, eps=EPS, weight_decay=WD, foreach=True)
        else:
            opt = BankAdamW(bank, T, lr=_lr(1), betas=BETAS, eps=EPS, weight_decay=WD)
        res = []
        for step, h in enumerate(hs, start=1):
            for grp in opt.param_groups:
                grp["lr"] = _lr(step)
            y, _ = layer(h, bank, return_losses=False)
            res.append(y.detach().cpu())
            (y.float() ** 2).mean().backward()
            params = [bank, *layer.parameters()]
            if kind == "torch":
                torch.nn.utils.clip_grad_norm_(params, 1e-3)
            else:
                clip_grad_norm_(params, 1e-3)
            opt.step()
            opt.zero_grad()
            layer.zero_grad(set_to_none=True)
        if kind != "torch":
            opt.flush()
        outs[kind] = (res, bank.detach().cpu())
    for i, (a, b) in enumerate(zip(outs["bank_adamw"][0], outs["torch"][0])):
        assert_rel(a, b, 1e-5, f"layer output at step {i + 1}")
    assert_rel(outs["bank_adamw"][1], outs["torch"][1], 1e-5, "bank after four steps")


def test_state_dict_round_trip_with_torch_adamw(dev):
    """BankAdamW's state_dict loads into torch.optim.AdamW (and back): one more step of each
    from the same state agrees."""
    from memory_amd.bank_optim import BankAdamW
    C, T, d = 6, 8, 64
    g0 = gen(61)
    bank = torch.nn.Parameter(torch.randn(C * T, d, generator=g0).to(dev))
    opt = BankAdamW(bank, T, lr=1e-2, betas=BETAS, eps=EPS, weight_decay=WD)
    for step in range(3):
        ch = torch.tensor([step, step + 2])
        opt.row_grad.add_(ch, torch.randn(2 * T, d, generator=g0).to(dev))
        opt.step()
        opt.zero_grad()
    sd = copy.deepcopy(opt.state_dict())   # state_dict hands out the live moments, as torch's does
    twin = torch.nn.Parameter(bank.detach().clone())
    ref = torch.optim.AdamW([twin], lr=1e-2, betas=BETAS, eps=EPS, weight_decay=WD)
    ref.load_state_dict(sd)
    g = torch.randn(C * T, d, generator=g0).to(dev)
    twin.grad = g.clone()
    ref.step()
    back = BankAdamW(torch.nn.Parameter(bank.detach().clone()), T, lr=1e-2, betas=BETAS, eps=EPS, weight_decay=WD)
    back.load_state_dict(ref.state_dict())
    bank.grad = g.clone()
    opt.step()
    assert_rel(bank.detach(), twin.detach(), 1e-6, "param after one more step")
    assert_rel(opt.exp_avg, ref.state[twin]["exp_avg"], 1e-6, "exp_avg")
    assert back.t == 4
    assert_rel(back.exp_avg_sq, ref.state[twin]["exp_avg_sq"], 0.0, "loaded exp_avg_sq")
