"""End-to-end parity of the module API (RoutedMemoryLayer = ChapterRouter +
MemoryCrossAttention on the fused sequence path) against the oracle's
sequence_memory_layer (float64 autograd), at BASELINE config 1:
B=2, L=128, d=256, 4 heads, bank 33 x 64, S=1 shared + k=4 routed, scale 2.5,
seed 0 (draw order h, bank, W_r, Wq, Wk, Wv, Wo; router bias 0; o_proj not zeroed).

Checked: chapter selection (bit-exact), output, and the gradients of h, the
bank, every projection, and the router weight and bias (the router gradient
flows only through the omega chain)."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, assert_rel

pytestmark = pytest.mark.gpu

C1 = dict(B=2, L=128, d=256, H=4, C=33, T=64, S=1, k=4, s=2.5)


def _config1_inputs(scale_w=0.02, L=None):
    torch.manual_seed(0)
    c = C1
    h = torch.randn(c["B"], L or c["L"], c["d"])
    bank = torch.randn(c["C"] * c["T"], c["d"]) * 0.02
    Wr = torch.randn(c["C"], c["d"]) * scale_w
    Wq, Wk, Wv, Wo = (torch.randn(c["d"], c["d"]) * scale_w for _ in range(4))
    br = torch.zeros(c["C"])
    return h, bank, Wr, br, Wq, Wk, Wv, Wo


def _layer(dev, dtype, Wr, br, Wq, Wk, Wv, Wo, normalize, strategy="sequence", window=None):
    from memory_amd.model import RoutedMemoryLayer
    c = C1
    layer = RoutedMemoryLayer(c["d"], c["H"], c["C"], c["T"], c["k"], num_shared_chapters=c["S"],
                              routed_scaling_factor=c["s"], normalize_shared_routed_before_mixing=normalize,
                              shared_routed_norm_eps=1e-6, routing_strategy=strategy, routing_window_size=window,
                              wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        layer.memory_attn.q_proj.weight.copy_(Wq)
        layer.memory_attn.k_proj.weight.copy_(Wk)
        layer.memory_attn.v_proj.weight.copy_(Wv)
        layer.memory_attn.o_proj.weight.copy_(Wo)
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj, layer.memory_attn.o_proj):
        m.to(dtype)
    return layer


@pytest.mark.parametrize("dtype,fused", [(torch.float32, "per-op"), (torch.bfloat16, "native"),
                                         (torch.bfloat16, "python"), (torch.bfloat16, "per-op")])
@pytest.mark.parametrize("normalize,strategy,window", [(False, "sequence", None), (True, "sequence", None),
                                                       (False, "sequence-rolling", 16)])
@pytest.mark.parametrize("Lq", [128, 96])
def test_config1_layer_forward_backward(gpu_device, monkeypatch, dtype, fused, normalize, strategy, window, Lq):
    """bf16 runs the whole-layer autograd function (memory_amd.seq_layer) with its native
    schedule (moc_seq_layer_fwd / _bwd; a normalised bank takes the Python-scheduled one) and
    with the Python-scheduled one, and the per-op functions; fp32 always takes the per-op path."""
    from memory_amd import seq_layer
    print(f"config1 layer dtype={dtype} fused={fused} normalize={normalize} strategy={strategy} L={Lq}", flush=True)
    monkeypatch.setattr(seq_layer, "NATIVE", fused == "native")
    dev = gpu_device
    c = C1
    # larger router / projection weights than the 0.02 recipe so that every gradient is well
    # above rounding noise (the recipe's o_proj of std 0.02 makes outputs ~1e-4)
    # (L = 96: rows of delta / lse padded to 128 in the native backward)
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _config1_inputs(scale_w=0.08, L=Lq)
    bank = bank * 25.0
    layer = _layer(dev, dtype, Wr, br, Wq, Wk, Wv, Wo, normalize, strategy, window)
    layer.fused = fused != "per-op"
    hg = h.to(dev, dtype).requires_grad_(True)
    bg = bank.to(dev, dtype).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    dO = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    (out.float() * dO.to(dev)).sum().backward()

    leaves = [t.double().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    if dtype != torch.float32:   # reference sees the same rounded activations / weights
        for i in (0, 1, 4, 5, 6, 7):
            leaves[i] = leaves[i].detach().to(dtype).double().requires_grad_(True)
    ref, det = O.sequence_memory_layer(*leaves, H=c["H"], HK=c["H"], C=c["C"], T=c["T"], S=c["S"], top_k=c["k"],
                                       routed_scale=c["s"], normalize=normalize, eps=1e-6, strategy=strategy,
                                       window=window, return_details=True)
    (ref * dO.double()).sum().backward()
    idx_star, _, _ = layer.route(hg.detach(), return_losses=False)
    assert torch.equal(idx_star.cpu(), det["idx_star"])
    assert_parity(out, ref, dtype, "out")
    names = ["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"]
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    for n, g, r in zip(names, got, leaves):
        assert_parity(g, r.grad, dtype, n)


def test_config1_recipe_scale_router_losses(gpu_device):
    """The exact BASELINE recipe (weights N(0, 0.02)): selection, output and the router losses."""
    from memory_amd.router import compute_total_router_loss
    dev = gpu_device
    c = C1
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _config1_inputs()
    layer = _layer(dev, torch.float32, Wr, br, Wq, Wk, Wv, Wo, False)
    out, losses = layer(h.to(dev), bank.to(dev), return_losses=True)
    ref, det = O.sequence_memory_layer(h.double(), bank.double(), Wr.double(), br.double(), Wq.double(),
                                       Wk.double(), Wv.double(), Wo.double(), H=c["H"], HK=c["H"], C=c["C"],
                                       T=c["T"], S=c["S"], top_k=c["k"], routed_scale=c["s"], return_details=True)
    idx_star, _, _ = layer.route(h.to(dev), return_losses=False)
    assert torch.equal(idx_star.cpu(), det["idx_star"]), "chapter selection differs from the oracle's"
    assert_parity(out, ref, torch.float32, "out")
    assert_rel(out, ref, 1e-4, "out")
    for k in ("load_balance", "auxiliary", "z_loss", "entropy"):
        assert_rel(losses[k].reshape(1), det["losses"][k].reshape(1), 1e-5, k)
    tot = compute_total_router_loss(losses, 0.01, 0.0, 0.001)
    rtot = O.compute_total_router_loss(det["losses"], 0.01, 0.0, 0.001)
    assert_rel(tot.reshape(1), rtot.reshape(1), 1e-5, "total router loss")


def test_native_stage_timing(gpu_device, monkeypatch):
    """The native layer's stage timing (moc_seq_layer_timing) times every stage of one forward +
    backward once, and is inert once disarmed."""
    from memory_amd import _lib, seq_layer
    monkeypatch.setattr(seq_layer, "NATIVE", True)
    dev = gpu_device
    h, bank, Wr, br, Wq, Wk, Wv, Wo = _config1_inputs(scale_w=0.08)
    layer = _layer(dev, torch.bfloat16, Wr, br, Wq, Wk, Wv, Wo, False)
    hg = h.to(dev, torch.bfloat16).requires_grad_(True)
    bg = bank.to(dev, torch.bfloat16).requires_grad_(True)

    def step():
        out, _ = layer(hg, bg, return_losses=False)
        out.float().sum().backward()

    step()
    torch.cuda.synchronize()
    _lib.seq_stage_timing(None, 2)
    try:
        step()
        torch.cuda.synchronize()
        st = _lib.seq_stage_read()
    finally:
        _lib.seq_stage_timing(None, 0)
    assert set(st) == set(_lib.seq_stage_names())
    for name, (ms, launches, dropped) in st.items():
        assert launches == 1 and dropped == 0 and 0.0 < ms < 100.0, (name, ms, launches, dropped)
    step()
    torch.cuda.synchronize()
    assert _lib.seq_stage_read() == {}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("normalize", [False, True])
def test_layer_128_token_chapters(gpu_device, dtype, normalize):
    """tokens_per_chapter = 128: each chapter runs as two 64-row chapters carrying its weight
    (ops.sub_chapters); selection, output and every gradient against the oracle's layer at
    T = 128 (the router's omega gradient is the sum over the two halves)."""
    from memory_amd.model import RoutedMemoryLayer
    print(f"layer T=128 dtype={dtype} normalize={normalize}", flush=True)
    dev = gpu_device
    B, Lq, d, H, C, T, S, k, s = 2, 96, 256, 4, 17, 128, 1, 4, 2.5
    g = torch.Generator().manual_seed(7)
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.5
    Wr = torch.randn(C, d, generator=g) * 0.08
    br = torch.zeros(C)
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) * 0.08 for _ in range(4))
    layer = RoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=S, routed_scaling_factor=s,
                              normalize_shared_routed_before_mixing=normalize, shared_routed_norm_eps=1e-6,
                              wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in zip((layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                           layer.memory_attn.o_proj), (Wq, Wk, Wv, Wo)):
            lin.weight.copy_(W)
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj, layer.memory_attn.o_proj):
        m.to(dtype)
    hg = h.to(dev, dtype).requires_grad_(True)
    bg = bank.to(dev, dtype).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    dO = torch.randn(out.shape, generator=torch.Generator().manual_seed(8))
    (out.float() * dO.to(dev)).sum().backward()

    leaves = [t.double().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    if dtype != torch.float32:
        for i in (0, 1, 4, 5, 6, 7):
            leaves[i] = leaves[i].detach().to(dtype).double().requires_grad_(True)
    ref, det = O.sequence_memory_layer(*leaves, H=H, HK=H, C=C, T=T, S=S, top_k=k, routed_scale=s,
                                       normalize=normalize, eps=1e-6, return_details=True)
    (ref * dO.double()).sum().backward()
    idx_star, _, _ = layer.route(hg.detach(), return_losses=False)
    assert torch.equal(idx_star.cpu(), det["idx_star"])
    assert_parity(out, ref, dtype, "out")
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    for n, gr, r in zip(["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"], got, leaves):
        assert_parity(gr, r.grad, dtype, n)
