"""model.split_rows (the token layer's shared / routed split of the bank) on the CPU: its
backward hands on a whole-bank gradient buffer only when the routed gradient was written into
the tail of a buffer marked for it; any other view of a full-size tensor -- here the one cat's
backward produces when a caller concatenates another n-row tensor with the routed rows -- is
copied, so no gradient row of another input is overwritten."""

import torch

from memory_amd.model import split_rows


def test_split_rows_gradient_through_cat_view():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(10, 4, generator=g, dtype=torch.float64, requires_grad=True)
    extra = torch.randn(3, 4, generator=g, dtype=torch.float64, requires_grad=True)
    a, b = split_rows(x, 3)
    z = torch.cat([extra, b])                   # same shape as x: b's gradient is a view of dz
    dz = torch.randn(10, 4, generator=g, dtype=torch.float64)
    (z * dz).sum().backward(retain_graph=True)
    assert torch.equal(extra.grad, dz[:3])
    want = torch.cat([torch.zeros(3, 4, dtype=torch.float64), dz[3:]])
    assert torch.equal(x.grad, want)
    # the head block's gradient, when it has one, lands in the head rows
    x.grad = None
    extra.grad = None
    ((a * 2.0).sum() + (z * dz).sum()).backward()
    assert torch.equal(extra.grad, dz[:3])
    assert torch.equal(x.grad, torch.cat([torch.full((3, 4), 2.0, dtype=torch.float64), dz[3:]]))


def test_split_rows_marked_tail_buffer_is_reused():
    x = torch.randn(6, 2, dtype=torch.float64, requires_grad=True)

    class Tail(torch.autograd.Function):
        @staticmethod
        def forward(ctx, t):
            return t.clone()

        @staticmethod
        def backward(ctx, gt):
            full = torch.empty(6, 2, dtype=gt.dtype)
            full._moc_rows_tail = 2
            tail = full[2:]
            tail.copy_(gt)
            return tail

    a, b = split_rows(x, 2)
    out = (Tail.apply(b) * 3.0).sum() + a.sum()
    out.backward()
    assert torch.equal(x.grad, torch.cat([torch.ones(2, 2, dtype=torch.float64),
                                          torch.full((4, 2), 3.0, dtype=torch.float64)]))
