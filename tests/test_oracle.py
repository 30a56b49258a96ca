"""Pins of the CPU oracle (no GPU).

Each test checks an oracle function against something other than its own
formula: a brute force, a closed form, a special case that reduces to a
textbook routine, a loop-form restatement of the reference's naive kernel
references, or finite differences (torch.autograd.gradcheck in float64).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O


@pytest.fixture(autouse=True)
def _float64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _rng(seed):
    g = torch.Generator().manual_seed(seed)
    return g


# ---------------------------------------------------------------- top-k / router

def test_topk_tie_rule_matches_bruteforce():
    g = _rng(0)
    x = torch.randint(0, 7, (9, 50), generator=g).double()   # many ties
    _, idx = O.topk_desc(x, 13)
    ref = O.topk_desc_numpy(x.numpy(), 13)
    assert np.array_equal(idx.numpy(), ref)


def test_route_sequence_logits_equals_probs_when_distinct():
    g = _rng(1)
    logits = torch.randn(6, 97, generator=g, dtype=torch.float32)
    for S in (0, 1, 3):
        i1, w1, p1 = O.route_sequence(logits, 8, S, select_by="logits")
        i2, w2, p2 = O.route_sequence(logits, 8, S, select_by="probs")
        assert torch.equal(i1, i2)
        assert torch.equal(w1, w2)
        # agrees with torch.topk where there are no ties
        p = p1.clone()
        if S:
            p[:, :S] = 0
            p = p / p.sum(-1, keepdim=True)
        assert torch.equal(torch.topk(p, 8, dim=-1).indices, i1)


def test_route_sequence_invariants():
    g = _rng(2)
    logits = torch.randn(5, 33, generator=g)
    idx, w, probs = O.route_sequence(logits, 4, 1)
    assert torch.allclose(w.sum(-1), torch.ones(5))
    assert (idx >= 1).all() and (idx < 33).all()
    sel = torch.gather(probs, -1, idx)
    assert (sel[:, :-1] >= sel[:, 1:]).all()
    # k = C - S selects every routed chapter
    idx_all, w_all, _ = O.route_sequence(logits, 32, 1)
    assert torch.equal(idx_all.sort(-1).values, torch.arange(1, 33).expand(5, -1))
    # the weights are a softmax over the selected logits (D1 cancels)
    assert torch.allclose(w, F.softmax(torch.gather(logits, -1, idx), dim=-1))


def test_route_token_level_matches_sequence_per_row():
    g = _rng(3)
    logits = torch.randn(2, 5, 40, generator=g)
    idx, w, _ = O.route_token_level(logits, 6, 2)
    i2, w2, _ = O.route_sequence(logits.reshape(10, 40), 6, 2)
    assert torch.equal(idx.reshape(10, 6), i2)
    assert torch.allclose(w.reshape(10, 6), w2)


def test_prepend_closed_form():
    idx = torch.tensor([[5, 9, 2, 7]])
    w = torch.tensor([[0.4, 0.3, 0.2, 0.1]])
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=33, num_shared_chapters=1,
                                       routed_scaling_factor=2.5)
    assert ci.tolist() == [[0, 5, 9, 2, 7]]
    assert abs(float(cw[0, 0]) - 1.0 / 3.5) < 1e-15
    assert torch.allclose(cw[0, 1:], 2.5 * w[0] / 3.5)


def test_rolling_pool_coefficients_and_special_cases():
    g = _rng(4)
    h = torch.randn(3, 11, 5, generator=g)
    for w in (1, 3, 4, 11, 50):
        direct = torch.stack([torch.stack([h[b, max(0, t - w + 1):t + 1].mean(0) for t in range(11)]).mean(0)
                              for b in range(3)])
        got = O.sequence_pool(h, "sequence-rolling", w)
        c = O.rolling_pool_coefficients(11, w)
        assert torch.allclose(got, direct)
        assert torch.allclose(torch.einsum("l,bld->bd", c, h), direct)
        assert abs(float(c.sum()) - 1.0) < 1e-12
    assert torch.allclose(O.sequence_pool(h, "sequence-rolling", 1), h.mean(1))
    assert torch.allclose(O.sequence_pool(h, "sequence-rolling", 11), O.sequence_pool(h, "sequence-rolling", None))


def test_router_losses_closed_forms():
    C, R, k = 16, 4, 3
    logits = torch.zeros(R, C)
    probs = F.softmax(logits, -1)
    idx = torch.arange(k).expand(R, -1)
    L = O.router_losses(logits, probs, idx, C)
    assert abs(float(L["load_balance"]) - k) < 1e-12          # C * sum f * (1/C)
    assert abs(float(L["z_loss"]) - math.log(C) ** 2) < 1e-12
    assert abs(float(L["entropy"]) - math.log(C)) < 1e-12
    assert abs(float(L["auxiliary"]) - (1.0 / C ** 2 - 1.0 / C) ** 2) < 1e-15
    tot = O.compute_total_router_loss(L, 0.01, 0.0, 0.001)
    assert abs(float(tot) - (0.01 * k + 0.001 * math.log(C) ** 2)) < 1e-12


def test_router_losses_one_hot_peaked_closed_form():
    """Rows whose probabilities are one-hot up to e^-60 at column c_r: mean_r p^2 per column is
    n_c / R (n_c = rows peaked at c), so auxiliary = mean_c (n_c / R - 1 / C)^2 -- a swap of the
    square and the row mean, (mean_r p)^2 = (n_c / R)^2, fails it; load balance =
    C sum_c f_c n_c / R with f_c = selections of c per row averaged over rows; entropy -> 0;
    z_loss = mean_r (60 + log(1 + (C - 1) e^-60))^2."""
    C, R = 7, 10
    peaks = torch.tensor([0, 0, 0, 1, 1, 2, 3, 3, 3, 3])
    logits = torch.zeros(R, C)
    logits[torch.arange(R), peaks] = 60.0
    probs = F.softmax(logits, -1)
    idx = torch.stack([peaks, (peaks + 2) % C], dim=1)          # each row selects its peak and one more
    L = O.router_losses(logits, probs, idx, C)
    n = torch.bincount(peaks, minlength=C).double()
    aux = float(((n / R - 1.0 / C) ** 2).mean())
    assert abs(float(L["auxiliary"]) - aux) < 1e-12
    swapped = float(((n / R) ** 2 - 1.0 / C).pow(2).mean())
    assert abs(swapped - aux) > 1e-3                           # the pin tells the two apart
    f = (torch.bincount(idx[:, 0], minlength=C) + torch.bincount(idx[:, 1], minlength=C)).double() / R
    assert abs(float(L["load_balance"]) - C * float((f * n / R).sum())) < 1e-12
    assert float(L["entropy"]) < 1e-20
    lse = 60.0 + math.log1p((C - 1) * math.exp(-60.0))
    assert abs(float(L["z_loss"]) - lse ** 2) < 1e-9


def test_sparse_unweighted_same_chapters_is_dense_attention():
    """Every token selecting the same chapters: the joint softmax over their keys is plain
    (textbook) attention over those rows, here torch's scaled_dot_product_attention."""
    g = _rng(17)
    B, Tq, HQ, HK, D, BS, M = 2, 9, 4, 2, 8, 4, 6
    q = torch.randn(B, Tq, HQ, D, generator=g)
    k = torch.randn(B, M * BS, HK, D, generator=g)
    v = torch.randn(B, M * BS, HK, D, generator=g)
    chosen = torch.tensor([4, 1, 3])
    idx = chosen.view(1, 1, 1, -1).expand(B, Tq, HK, 3)
    sc = 0.37
    got = O.sparse_attention_unweighted(q, k, v, idx, BS, sc)
    rows = (chosen.view(-1, 1) * BS + torch.arange(BS)).reshape(-1)
    kk = k[:, rows].repeat_interleave(HQ // HK, dim=2).transpose(1, 2)     # (B, HQ, keys, D)
    vv = v[:, rows].repeat_interleave(HQ // HK, dim=2).transpose(1, 2)
    want = F.scaled_dot_product_attention(q.transpose(1, 2), kk, vv, scale=sc).transpose(1, 2)
    assert torch.allclose(got, want, atol=1e-12)


def test_select_from_probs_equals_route():
    g = _rng(5)
    logits = torch.randn(4, 21, generator=g)
    probs = F.softmax(logits, -1)
    i1, w1 = O.select_routed_chapters_from_probs(probs, 5, 1)
    i2, w2, _ = O.route_sequence(logits, 5, 1, select_by="probs")
    assert torch.equal(i1, i2) and torch.allclose(w1, w2)


# ---------------------------------------------------------------- gather / normalise

def test_gather_index_arithmetic():
    g = _rng(6)
    bank = torch.randn(7 * 4, 3, generator=g)
    idx = torch.tensor([[2, 0, 6], [5, 5, 1]])
    mem, flat = O.gather_chapters(bank, idx, 4)
    for b in range(2):
        for s in range(3):
            for j in range(4):
                row = int(idx[b, s]) * 4 + j
                assert int(flat[b, s * 4 + j]) == row
                assert torch.equal(mem[b, s * 4 + j], bank[row])


def test_normalize_noop_cases_and_rms():
    g = _rng(7)
    mem = torch.randn(2, 12, 8, generator=g)
    assert torch.equal(O.normalize_shared_routed(mem, num_shared_chapters=0, tokens_per_chapter=4,
                                                 norm_type="rms", eps=1e-6), mem)
    assert torch.equal(O.normalize_shared_routed(mem, num_shared_chapters=3, tokens_per_chapter=4,
                                                 norm_type="rms", eps=1e-6), mem)
    out = O.normalize_shared_routed(mem, num_shared_chapters=1, tokens_per_chapter=4,
                                    norm_type="rms", eps=0.0)
    assert torch.allclose(out.pow(2).mean(-1), torch.ones(2, 12))
    ln = O.normalize_shared_routed(mem, num_shared_chapters=1, tokens_per_chapter=4,
                                   norm_type="layernorm", eps=0.0)
    assert torch.allclose(ln.mean(-1), torch.zeros(2, 12), atol=1e-12)


# ---------------------------------------------------------------- attention

def _weights(g, d, H, HK, dh=None):
    dh = dh or d // H
    Wq = torch.randn(H * dh, d, generator=g) * 0.1
    Wk = torch.randn(HK * dh, d, generator=g) * 0.1
    Wv = torch.randn(HK * dh, d, generator=g) * 0.1
    Wo = torch.randn(d, H * dh, generator=g) * 0.1
    return Wq, Wk, Wv, Wo


def test_cross_attention_vs_explicit_loops():
    g = _rng(8)
    B, L, N, d, H, HK = 2, 3, 5, 8, 4, 2
    h = torch.randn(B, L, d, generator=g)
    mem = torch.randn(B, N, d, generator=g)
    Wq, Wk, Wv, Wo = _weights(g, d, H, HK)
    out = O.cross_attention(h, mem, Wq, Wk, Wv, Wo, H, HK)
    dh = d // H
    ref = torch.zeros(B, L, d)
    for b in range(B):
        heads = []
        for hq in range(H):
            hk = hq // (H // HK)
            q = h[b] @ Wq[hq * dh:(hq + 1) * dh].T
            k = mem[b] @ Wk[hk * dh:(hk + 1) * dh].T
            v = mem[b] @ Wv[hk * dh:(hk + 1) * dh].T
            s = q @ k.T / math.sqrt(dh)
            e = torch.exp(s - s.max(-1, keepdim=True).values)
            heads.append((e / e.sum(-1, keepdim=True)) @ v)
        ref[b] = torch.cat(heads, -1) @ Wo.T
    assert torch.allclose(out, ref, atol=1e-12)


def _seq_setup(seed=9, B=2, L=6, d=16, H=2, HK=2, C=9, T=4):
    g = _rng(seed)
    h = torch.randn(B, L, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.5
    Wr = torch.randn(C, d, generator=g) * 0.5
    br = torch.zeros(C)
    Wq, Wk, Wv, Wo = _weights(g, d, H, HK)
    return h, bank, Wr, br, Wq, Wk, Wv, Wo


@pytest.mark.parametrize("normalize", [False, True])
def test_semantics_A_omega_in_attention_equivalence(normalize):
    """(omega x) W = omega (x W): scaling logits and values by omega over
    unweighted projections equals the reference chain that weights rows first."""
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _seq_setup()
    H, HK, C, T, S, k, s = 2, 2, 9, 4, 1, 3, 2.5
    out, det = O.sequence_memory_layer(h, bank, Wr, br, Wq, Wk, Wv, Wo, H=H, HK=HK, C=C, T=T,
                                       S=S, top_k=k, routed_scale=s, normalize=normalize,
                                       eps=1e-5, return_details=True)
    B, L, d = h.shape
    dh = d // H
    X, _ = O.gather_chapters(bank, det["idx_star"], T)
    if normalize:
        X = O.rms_norm(X, 1e-5)
    om = det["omega"].repeat_interleave(T, dim=1)          # (B, N)
    q = (h @ Wq.T).view(B, L, H, dh)
    kh = (X @ Wk.T).view(B, -1, HK, dh)
    vh = (X @ Wv.T).view(B, -1, HK, dh)
    sc = torch.einsum("blhd,bnhd->bhln", q, kh) * om[:, None, None, :] / math.sqrt(dh)
    p = F.softmax(sc, -1)
    a = torch.einsum("bhln,bnhd->blhd", p * om[:, None, None, :], vh).reshape(B, L, d)
    assert torch.allclose(a @ Wo.T, out, atol=1e-12)


def test_semantics_A_all_chapters_equal_weight_is_dense():
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _seq_setup(C=5)
    # S=0, k=C, router weights forced equal -> omega = 1/C for every chapter
    C, T = 5, 4
    idx = torch.arange(C).expand(2, -1)
    w = torch.full((2, C), 1.0 / C)
    mem, _ = O.gather_chapters(bank, idx, T)
    mem = O.weight_memory(mem, w, T)
    out = O.cross_attention(h, mem, Wq, Wk, Wv, Wo, 2, 2)
    dense = O.cross_attention(h, bank / C, Wq, Wk, Wv, Wo, 2, 2)
    assert torch.allclose(out, dense, atol=1e-12)


def test_sequence_layer_gradcheck():
    """Finite differences pin the autograd of the whole routed layer (selection fixed)."""
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _seq_setup(seed=10, B=2, L=3, d=8, H=2, HK=1, C=6, T=2)
    args = [t.clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]

    def f(*a):
        return O.sequence_memory_layer(*a, H=2, HK=1, C=6, T=2, S=1, top_k=2, routed_scale=2.5,
                                       normalize=True, eps=1e-5)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-7)


def test_router_weight_grad_closed_form():
    """d(logits) of omega(logits) equals the restricted softmax Jacobian."""
    g = _rng(11)
    R, C, S, k, s = 3, 12, 1, 4, 2.5
    z = torch.randn(R, C, generator=g, requires_grad=True)
    idx, w, _ = O.route_sequence(z, k, S)
    _, om = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S,
                                      routed_scaling_factor=s)
    gom = torch.randn(R, S + k, generator=g)
    (om * gom).sum().backward()
    gw = gom[:, S:] * s / (S + s)
    what = w.detach()
    dz = torch.zeros(R, C)
    dz.scatter_(1, idx, what * (gw - (what * gw).sum(-1, keepdim=True)))
    assert torch.allclose(z.grad, dz, atol=1e-12)


# ---------------------------------------------------------------- token-level kernels

def _sparse_inputs(seed, B=1, TQ=5, HQ=4, HK=2, D=8, M=6, BS=4, S=3):
    g = _rng(seed)
    q = torch.randn(B, TQ, HQ, D, generator=g)
    k = torch.randn(B, M * BS, HK, D, generator=g)
    v = torch.randn(B, M * BS, HK, D, generator=g)
    idx = torch.stack([torch.stack([torch.randperm(M, generator=g)[:S] for _ in range(HK)])
                       for _ in range(B * TQ)]).view(B, TQ, HK, S)
    w = torch.rand(B, TQ, S, generator=g)
    w = w / w.sum(-1, keepdim=True)
    return q, k, v, idx, w, BS


def test_sparse_weighted_vs_naive_loop():
    q, k, v, idx, w, BS = _sparse_inputs(12)
    sc = 0.3
    assert torch.allclose(O.sparse_attention_weighted(q, k, v, idx, w, BS, sc),
                          O.naive_reference_weighted(q, k, v, idx, w, BS, sc), atol=1e-12)


def test_sparse_unweighted_vs_naive_loop():
    q, k, v, idx, w, BS = _sparse_inputs(13)
    assert torch.allclose(O.sparse_attention_unweighted(q, k, v, idx, BS, 0.3),
                          O.naive_reference_unweighted(q, k, v, idx, BS, 0.3), atol=1e-12)


def test_sparse_joint_bias_vs_naive_and_equal_weight_case():
    q, k, v, idx, w, BS = _sparse_inputs(14)
    assert torch.allclose(O.sparse_attention_joint_bias(q, k, v, idx, w, BS, 0.3),
                          O.naive_reference_weighted_joint_bias(q, k, v, idx, w, BS, 0.3), atol=1e-12)
    eq = torch.full_like(w, 1.0 / w.shape[-1])
    assert torch.allclose(O.sparse_attention_joint_bias(q, k, v, idx, eq, BS, 0.3),
                          O.sparse_attention_unweighted(q, k, v, idx, BS, 0.3), atol=1e-12)


def test_sparse_block_weighted_vs_loop_and_ones():
    q, k, v, idx, w, BS = _sparse_inputs(15)
    g = _rng(16)
    bw = torch.rand(idx.shape, generator=g)
    assert torch.allclose(O.sparse_attention_block_weighted(q, k, v, idx, bw, BS, 0.3),
                          O.naive_reference_block_weighted(q, k, v, idx, bw, BS, 0.3), atol=1e-12)
    assert torch.allclose(O.sparse_attention_block_weighted(q, k, v, idx, torch.ones_like(bw), BS, 0.3),
                          O.sparse_attention_unweighted(q, k, v, idx, BS, 0.3), atol=1e-12)


def test_weighted_single_chapter_is_plain_attention():
    q, k, v, idx, w, BS = _sparse_inputs(17, S=1)
    out = O.sparse_attention_weighted(q, k, v, idx, torch.ones_like(w), BS, 0.125)
    ref = torch.zeros_like(out)
    for t in range(q.shape[1]):
        for hq in range(q.shape[2]):
            hk = hq // 2
            c0 = int(idx[0, t, hk, 0]) * BS
            kk, vv = k[0, c0:c0 + BS, hk], v[0, c0:c0 + BS, hk]
            p = F.softmax(q[0, t, hq] @ kk.T * 0.125, -1)
            ref[0, t, hq] = p @ vv
    assert torch.allclose(out, ref, atol=1e-12)


def test_token_layer_shared_branch_is_dense_attention():
    g = _rng(18)
    B, L, d, H, C, T = 1, 4, 8, 2, 5, 4
    h = torch.randn(B, L, d, generator=g)
    bank = torch.randn(C * T, d, generator=g)
    Wq, Wk, Wv, Wo = _weights(g, d, H, H)
    pre = O.token_routed_preproj(h, bank[:T], None, torch.zeros(B, L, 0, dtype=torch.long), None,
                                 T, 2.5, Wq, Wk, Wv, H, H)
    dense = O.cross_attention(h, bank[:T], Wq, Wk, Wv, None, H, H, return_preproj=True)
    assert torch.allclose(pre, dense, atol=1e-12)


def test_token_layer_gradcheck():
    g = _rng(19)
    B, L, d, H, C, T = 1, 3, 8, 2, 5, 2
    args = [torch.randn(B, L, d, generator=g), torch.randn(C * T, d, generator=g),
            torch.randn(C, d, generator=g), torch.zeros(C)] + list(_weights(g, d, H, H))
    args = [a.requires_grad_(True) for a in args]

    def f(*a):
        return O.token_memory_layer(*a, H=H, HK=H, C=C, T=T, S=1, top_k=2, routed_scale=2.5)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-7)


def test_decode_is_L1_sequence_layer():
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _seq_setup(seed=20, L=1)
    out, det = O.sequence_memory_layer(h, bank, Wr, br, Wq, Wk, Wv, Wo, H=2, HK=2, C=9, T=4, S=1,
                                       top_k=3, routed_scale=2.5, return_details=True)
    dec = O.decode_step(h, bank, det["idx_star"], det["omega"], Wq, Wk, Wv, Wo, H=2, HK=2, T=4)
    assert torch.allclose(out, dec, atol=1e-12)


def test_moe_with_routing_single_chapter_equals_cross_attention():
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _seq_setup(seed=21)
    idx = torch.tensor([[3], [7]])
    out = O.moe_with_routing(h, bank, idx, torch.ones(2, 1), 4, Wq, Wk, Wv, Wo, 2, 2)
    mem, _ = O.gather_chapters(bank, idx, 4)
    assert torch.allclose(out, O.cross_attention(h, mem, Wq, Wk, Wv, Wo, 2, 2), atol=1e-12)


@pytest.mark.parametrize("foreach", [False, True])
def test_adamw_step_matches_torch_adamw(foreach):
    """The oracle's AdamW against torch.optim.AdamW itself (the reference's optimizer, a library
    routine) over several steps with a changing lr, weight decay and rows whose gradient is zero."""
    g0 = _rng(11)
    p = torch.randn(7, 5, generator=g0)
    ref = p.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=foreach)
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for step in range(1, 7):
        lr = 1e-2 * (0.5 + 0.1 * step)
        for grp in opt.param_groups:
            grp["lr"] = lr
        g = torch.randn(7, 5, generator=g0)
        g[step % 7] = 0.0                       # a row without gradient this step
        ref.grad = g.clone()
        opt.step()
        O.adamw_step(p, g, m, v, step, lr, (0.9, 0.95), 1e-8, 0.1)
        st = opt.state[ref]
        assert torch.allclose(p, ref.detach(), rtol=0, atol=1e-13)
        assert torch.allclose(m, st["exp_avg"], rtol=0, atol=1e-13)
        assert torch.allclose(v, st["exp_avg_sq"], rtol=0, atol=1e-13)


def test_adamw_first_step_closed_form():
    """Step 1: m/bc1 = g and sqrt(v/bc2) = |g|, so p1 = p0 (1 - lr wd) - lr g / (|g| + eps)."""
    g0 = _rng(12)
    p0 = torch.randn(20, generator=g0)
    g = torch.randn(20, generator=g0)
    p, m, v = p0.clone(), torch.zeros(20), torch.zeros(20)
    lr, wd, eps = 3e-3, 0.1, 1e-8
    O.adamw_step(p, g, m, v, 1, lr, (0.9, 0.95), eps, wd)
    assert torch.allclose(p, p0 * (1 - lr * wd) - lr * g / (g.abs() + eps), rtol=0, atol=1e-14)


@pytest.mark.parametrize("max_norm", [0.5, 1e3])
def test_clip_grad_norm_matches_torch(max_norm):
    g0 = _rng(13)
    ps = [torch.randn(s, generator=g0).requires_grad_(True) for s in ((4, 3), (5,), (2, 2, 2))]
    grads = [torch.randn(pp.shape, generator=g0) for pp in ps]
    for pp, gg in zip(ps, grads):
        pp.grad = gg.clone()
    total_ref = torch.nn.utils.clip_grad_norm_(ps, max_norm)
    total = O.clip_grad_norm(grads, max_norm)
    assert torch.allclose(total, total_ref, rtol=1e-14)
    for pp, gg in zip(ps, grads):
        assert torch.allclose(gg, pp.grad, rtol=1e-14, atol=0)


def test_block_rms_norm_matches_torch_rms_norm():
    """The reference's RMSNorm module restated, against torch's own rms_norm (a library
    routine with the same definition) and a closed form: a constant row c gives sign(c) * w."""
    g0 = _rng(21)
    x = torch.randn(5, 7, 24, generator=g0)
    w = torch.randn(24, generator=g0)
    ref = F.rms_norm(x, (24,), w, 1e-6)
    assert torch.allclose(O.block_rms_norm(x, w, 1e-6), ref, rtol=1e-12, atol=1e-12)
    c = torch.full((3, 24), -2.5)
    assert torch.allclose(O.block_rms_norm(c, w, 0.0), -w.expand(3, 24), rtol=1e-14)


def test_memory_sublayer_is_residual_plus_cross_attention():
    """With a zero output projection the sublayer is the identity (the wo_init_zero start of
    memory_attention.py:140-143), and with LayerNorm of unit weight / zero bias it equals the
    residual plus attention over standardised rows."""
    g0 = _rng(22)
    B, L, N, d, H = 2, 5, 8, 16, 2
    h = torch.randn(B, L, d, generator=g0)
    mem = torch.randn(B, N, d, generator=g0)
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g0) * 0.2 for _ in range(4))
    out = O.memory_sublayer(h, torch.ones(d), None, 1e-6, True, mem, Wq, Wk, Wv, torch.zeros(d, d), H, H)
    assert torch.equal(out, h)
    out = O.memory_sublayer(h, torch.ones(d), torch.zeros(d), 1e-5, False, mem, Wq, Wk, Wv, Wo, H, H)
    xs = (h - h.mean(-1, keepdim=True)) / torch.sqrt(h.var(-1, unbiased=False, keepdim=True) + 1e-5)
    assert torch.allclose(out, h + O.cross_attention(xs, mem, Wq, Wk, Wv, Wo, H, H), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ inference routing (decode)

def test_masked_mean_special_cases():
    """model.py:468-493: no mask = mean; a one-hot mask picks that position; an all-zero row is
    0 (count clamped to 1); a longer mask is aligned on its rightmost columns."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 5, 4, generator=g, dtype=torch.float64)
    torch.testing.assert_close(O.masked_mean(x, None), x.mean(1))
    torch.testing.assert_close(O.masked_mean(x, torch.ones(3, 5)), x.mean(1))
    oh = torch.zeros(3, 5)
    oh[0, 2] = oh[1, 4] = 1
    got = O.masked_mean(x, oh)
    torch.testing.assert_close(got[0], x[0, 2])
    torch.testing.assert_close(got[1], x[1, 4])
    assert torch.equal(got[2], torch.zeros(4, dtype=torch.float64))
    long = torch.cat([torch.zeros(3, 7), torch.ones(3, 5)], dim=1)
    torch.testing.assert_close(O.masked_mean(x, long), x.mean(1))


def test_inference_route_windows_brute_force():
    """The pooled router input of every strategy over a prefill and 5 steps, against brute force:
    rolling = mean of the last W states of (prompt + generated so far); hybrid = the prompt's mean
    at prefill, then the rolling window; sequence / sequence-rolling at a step = the token itself."""
    g = torch.Generator().manual_seed(4)
    B, P, d, C, W = 2, 7, 8, 10, 4
    Wr = torch.randn(C, d, generator=g, dtype=torch.float64)
    br = torch.randn(C, generator=g, dtype=torch.float64)
    prompt = torch.randn(B, P, d, generator=g, dtype=torch.float64)
    toks = [torch.randn(B, 1, d, generator=g, dtype=torch.float64) for _ in range(5)]
    kw = dict(top_k=3, num_shared=1, num_chapters=C, routed_scale=2.5, window=W)
    for strat in ("sequence", "sequence-rolling", "rolling", "hybrid"):
        hist = [prompt[:, i:i + 1] for i in range(P)]
        pooled, logits, ci, cw, cache = O.inference_route(strat, prompt, None, Wr, br, prefill=True, **kw)
        if strat in ("sequence", "hybrid"):
            torch.testing.assert_close(pooled, prompt.mean(1))
        elif strat == "rolling":
            torch.testing.assert_close(pooled, prompt[:, -W:].mean(1))
        else:
            torch.testing.assert_close(pooled, O.sequence_pool(prompt, "sequence-rolling", W))
        torch.testing.assert_close(logits, pooled @ Wr.T + br)
        assert ci.shape == (B, 4) and torch.equal(ci[:, 0], torch.zeros(B, dtype=torch.long))
        torch.testing.assert_close(cw.sum(-1), torch.ones(B, dtype=torch.float64))
        for t in toks:
            hist.append(t)
            pooled, _, ci, cw, cache = O.inference_route(strat, t, cache, Wr, br, **kw)
            if strat in ("rolling", "hybrid"):
                torch.testing.assert_close(pooled, torch.cat(hist[-W:], dim=1).mean(1))
                assert cache.shape[1] == W
            else:
                torch.testing.assert_close(pooled, t[:, 0])


def test_attention_weights_consistent_with_attention():
    """The returned weights are the probabilities ``attention`` mixes the values with (pinned
    there against SDPA): weights @ v (GQA expanded) == attention(q, k, v), rows sum to 1."""
    g = torch.Generator().manual_seed(5)
    B, L, N, H, HK, Dh = 2, 5, 128, 4, 2, 8
    d = H * Dh
    h = torch.randn(B, L, d, generator=g, dtype=torch.float64)
    mem = torch.randn(B, N, d, generator=g, dtype=torch.float64)
    Wq = torch.randn(d, d, generator=g, dtype=torch.float64)
    Wk = torch.randn(HK * Dh, d, generator=g, dtype=torch.float64)
    Wv = torch.randn(HK * Dh, d, generator=g, dtype=torch.float64)
    P = O.attention_weights(h, mem, Wq, Wk, H, HK)
    assert P.shape == (B, H, L, N)
    torch.testing.assert_close(P.sum(-1), torch.ones(B, H, L, dtype=torch.float64))
    q, k, v = O.compute_qkv(h, mem, Wq, Wk, Wv, H, HK)
    ve = v.repeat_interleave(H // HK, dim=2).transpose(1, 2)
    torch.testing.assert_close(torch.matmul(P, ve).transpose(1, 2), O.attention(q, k, v))
