"""Row-sparse gradient and AdamW for the chapter bank.

The reference keeps the bank as one fp32 parameter (``StandardMemoryBank.memory``,
memory_transformer/memory_bank.py:62) and trains it like every other parameter
(training/trainer.py:309-392): the gather's autograd gives a dense (N_m, d) gradient, zero
except the selected chapters' rows; ``accelerator.clip_grad_norm_`` (trainer.py:876-882)
folds it into the global norm; ``torch.optim.AdamW`` (param group "memory_bank", weight decay
0.1 in configs/base_small_run2.yaml:159) steps all N_m * d elements every step.

Here:

* ``RowSparseBankGrad`` — the bank's gradient as rows of the chapters that were read: the
  sequence-level layer's backward accumulates them in fp32 (``moc_bank_grad_accumulate``)
  instead of materialising the dense gradient; several layers sharing the bank and several
  micro-batches add up, first contributions are stored (no zero fill).
* ``BankAdamW`` — ``torch.optim.AdamW``'s update for the bank on one HIP kernel.  Dense
  gradients (``bank.grad``) are stepped in one pass; row-sparse gradients step only the touched
  chapters, and every other chapter is brought forward *exactly* — its zero-gradient steps
  (moment decay, weight decay, bias corrections with each step's lr) replayed in registers —
  when a layer next reads it (the layers call ``catch_up`` on their plan's chapters before the
  gather) or on ``flush()`` (``state_dict`` flushes).  An optional bf16 mirror of the bank is
  kept current for the forward kernels.
* ``clip_grad_norm_`` — ``torch.nn.utils.clip_grad_norm_`` (norm_type 2) that also counts the
  row-sparse bank gradients of the parameters it is given; the clip coefficient reaches the
  bank's step as a device scalar (no host synchronisation).
"""

from __future__ import annotations

import math
from typing import Iterable, Optional

import torch

from . import _lib as L
from ._lib import call, ptr, stream_ptr


def _chapters_of(bank: torch.Tensor, tokens_per_chapter: int) -> int:
    T = int(tokens_per_chapter)
    if bank.dim() != 2 or T <= 0 or bank.shape[0] % T != 0:
        raise ValueError(f"bank of shape {tuple(bank.shape)} is not a whole number of {T}-row chapters")
    return bank.shape[0] // T


class RowSparseBankGrad:
    """fp32 gradient rows of the chapters read since the last ``zero_()``.

    ``acc`` has the bank's shape but only the rows of chapters whose tag equals the current
    epoch are valid; attaching sets ``bank._moc_row_grad`` so that the routed layers send the
    bank gradient here (their autograd returns no dense bank gradient)."""

    def __init__(self, bank: torch.Tensor, tokens_per_chapter: int, attach: bool = True):
        L.require_gpu(bank)
        self.T = int(tokens_per_chapter)
        self.C = _chapters_of(bank, self.T)
        self.d = bank.shape[1]
        dev = bank.device
        self.acc = torch.empty(bank.shape, device=dev, dtype=torch.float32)
        self.chap_epoch = torch.full((self.C,), -1, device=dev, dtype=torch.int32)
        self.epoch = 0
        self.max_touched = 0            # host bound on the chapters holding rows this epoch
        self.scale: Optional[torch.Tensor] = None   # clip coefficient (device scalar) or None
        self._list = torch.empty(self.C, device=dev, dtype=torch.int32)
        self._n = torch.zeros(1, device=dev, dtype=torch.int32)
        self._list_epoch = None
        if attach:
            bank._moc_row_grad = self

    @property
    def has_rows(self) -> bool:
        return self.max_touched > 0

    def accumulate(self, dX: torch.Tensor, bank_read: torch.Tensor, uniq, n_uniq, max_u: int, csr_off=None,
                   csr_edge=None, mean=None, rstd=None, norm: int = L.MOC_NORM_NONE) -> None:
        """Add the gradient rows of one plan (``moc_bank_scatter``'s inputs) for this epoch."""
        if max_u == 0:
            return
        fresh = torch.empty(max_u, device=self.acc.device, dtype=torch.int32)
        call("moc_bank_grad_accumulate", L.dtype_code(dX.dtype), ptr(dX), ptr(bank_read), L.dtype_code(bank_read.dtype),
             self.d, self.T, ptr(uniq), ptr(n_uniq), max_u, ptr(csr_off), ptr(csr_edge), ptr(mean), ptr(rstd), norm,
             self.epoch, ptr(self.chap_epoch), ptr(fresh), ptr(self.acc), stream_ptr(self.acc.device))
        self.max_touched = min(self.C, self.max_touched + int(max_u))
        self._list_epoch = None

    def add_(self, chapters: torch.Tensor, rows: torch.Tensor) -> None:
        """Add explicit gradient rows: ``rows`` (len(chapters) * T, d) for the distinct
        ``chapters`` (int tensor)."""
        chapters = chapters.to(device=self.acc.device, dtype=torch.int32).contiguous()
        n = chapters.numel()
        if rows.shape != (n * self.T, self.d):
            raise ValueError(f"rows of shape {tuple(rows.shape)}, expected {(n * self.T, self.d)}")
        if n and torch.unique(chapters).numel() != n:
            raise ValueError("chapters must be distinct")
        if n and (int(chapters.min()) < 0 or int(chapters.max()) >= self.C):
            raise ValueError(f"chapter ids must lie in [0, {self.C})")
        rows = rows.contiguous()
        if rows.dtype not in (torch.float32, torch.bfloat16):
            rows = rows.float()
        n_dev = torch.full((1,), n, device=self.acc.device, dtype=torch.int32)
        self.accumulate(rows, rows.new_empty(1, self.d), chapters, n_dev, n)

    def touched(self):
        """(list, n): the chapters holding rows this epoch, ascending, on the device."""
        if self._list_epoch != self.epoch:
            call("moc_bank_touched", ptr(self.chap_epoch), self.C, self.epoch, ptr(self._list), ptr(self._n),
                 stream_ptr(self.acc.device))
            self._list_epoch = self.epoch
        return self._list, self._n

    def sqnorm(self) -> torch.Tensor:
        """Sum of squares of the gradient rows (fp32 device scalar, fixed summation order)."""
        out = torch.zeros(1, device=self.acc.device, dtype=torch.float32)
        if not self.has_rows:
            return out
        lst, n = self.touched()
        chunk = self.T * self.d
        ws_bytes = L.query("moc_bank_sqnorm_workspace", self.max_touched, chunk)
        ws = torch.empty(max(1, ws_bytes // 4), device=self.acc.device, dtype=torch.float32)
        call("moc_bank_sqnorm", ptr(self.acc), ptr(lst), ptr(n), self.max_touched, chunk, ptr(ws), ws_bytes,
             ptr(out), stream_ptr(self.acc.device))
        return out

    def to_dense(self) -> torch.Tensor:
        """The dense (N_m, d) gradient these rows stand for (for inspection and tests)."""
        out = torch.zeros_like(self.acc)
        if self.has_rows:
            lst, n = self.touched()
            ch = lst[: int(n.item())].long()
            rows = (ch[:, None] * self.T + torch.arange(self.T, device=ch.device)[None, :]).reshape(-1)
            out[rows] = self.acc[rows]
            if self.scale is not None:
                out[rows] *= self.scale
        return out

    def zero_(self) -> None:
        self.epoch += 1
        self.max_touched = 0
        self.scale = None
        self._list_epoch = None


class BankAdamW(torch.optim.Optimizer):
    """``torch.optim.AdamW`` (amsgrad off) for one fp32 chapter bank, on HIP kernels.

    ``BankAdamW(bank, tokens_per_chapter, lr, betas, eps, weight_decay, mirror_dtype=None,
    row_sparse=True)``.  With ``row_sparse`` a ``RowSparseBankGrad`` is attached to the bank
    (``self.row_grad``) and the routed layers accumulate into it; ``bank.grad`` (dense, e.g. from
    the token-level layer, which projects every chapter) is stepped as well.  The layers call
    ``catch_up`` before reading chapters; anything else that reads the bank must call
    ``flush()`` first (``state_dict()`` does).  ``mirror`` (bf16) follows the bank for the
    forward kernels when ``mirror_dtype=torch.bfloat16``.

    As in torch, a step in which the bank has no gradient at all does not advance it."""

    def __init__(self, bank: torch.nn.Parameter, tokens_per_chapter: int, lr: float = 1e-3,
                 betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 1e-2,
                 mirror_dtype: Optional[torch.dtype] = None, row_sparse: bool = True):
        L.require_gpu(bank)
        if bank.dtype != torch.float32 or not bank.is_contiguous():
            raise ValueError("BankAdamW steps a contiguous fp32 bank (the reference's master copy)")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"invalid betas {betas}")
        super().__init__([bank], dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))
        self.bank = bank
        self.T = int(tokens_per_chapter)
        self.C = _chapters_of(bank, self.T)
        dev = bank.device
        self.chunk = self.T * bank.shape[1]
        nchunk = int(L.query("moc_bank_chunk_count", self.chunk))
        self.exp_avg = torch.zeros_like(bank, memory_format=torch.contiguous_format)
        self.exp_avg_sq = torch.zeros_like(bank, memory_format=torch.contiguous_format)
        self.tags = torch.zeros(self.C * nchunk, device=dev, dtype=torch.int32)
        self.hist = torch.zeros(1024, 4, device=dev, dtype=torch.float32)
        self.t = 0
        self.mirror = None
        if mirror_dtype is not None:
            if mirror_dtype != torch.bfloat16:
                raise ValueError("the bank mirror must be bfloat16")
            self.mirror = bank.detach().to(torch.bfloat16)
        self.row_grad = RowSparseBankGrad(bank, self.T) if row_sparse else None
        bank._moc_bank_opt = self

    # ------------------------------------------------------------------ reads
    def read_view(self, compute_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """The tensor the forward kernels read: the bf16 mirror if there is one and the
        layer computes in bf16 (None: any dtype), else the fp32 bank."""
        if self.mirror is not None and compute_dtype != torch.float32:
            return self.mirror
        return self.bank

    def _run(self, grad, list_, n_list, max_list, step, scalars, grad_scale=None):
        g = self.param_groups[0]
        b1, b2 = g["betas"]
        call("moc_bank_adamw", ptr(self.bank), ptr(self.mirror), L.MOC_BF16, ptr(self.exp_avg), ptr(self.exp_avg_sq),
             ptr(grad), ptr(grad_scale), ptr(list_), ptr(n_list), max_list, self.C, self.chunk, ptr(self.tags),
             ptr(self.hist), self.hist.shape[0], step, *scalars, b1, b2, g["eps"], stream_ptr(self.bank.device))

    def catch_up(self, chapters: Optional[torch.Tensor] = None, n_chapters: Optional[torch.Tensor] = None,
                 max_chapters: Optional[int] = None) -> None:
        """Bring the given chapters (int32 device list with its device count, at most
        ``max_chapters``; None = every chapter) to the last completed step."""
        if self.t == 0:
            return
        with torch.no_grad():
            if chapters is None:
                self._run(None, None, None, 0, self.t, (1.0, 0.0, 1.0))
            else:
                self._run(None, chapters, n_chapters, int(max_chapters), self.t, (1.0, 0.0, 1.0))

    def flush(self) -> None:
        """Bring every chapter to the last completed step."""
        self.catch_up(None)

    def sync_mirror(self) -> None:
        """After the bank's values were written outside the optimizer (a checkpoint load, after
        ``flush()``): the bf16 mirror the kernels read is refreshed from the bank."""
        if self.mirror is not None:
            with torch.no_grad():
                self.mirror.copy_(self.bank.detach())

    # ------------------------------------------------------------------ step
    def _step_scalars(self, t: int):
        g = self.param_groups[0]
        lr, wd = g["lr"], g["weight_decay"]
        b1, b2 = g["betas"]
        if isinstance(lr, torch.Tensor):
            lr = float(lr)
        bc1 = 1 - b1 ** t
        bc2 = 1 - b2 ** t
        return (1 - lr * wd, -(lr / bc1), math.sqrt(bc2))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        dense = self.bank.grad
        sparse = self.row_grad if (self.row_grad is not None and self.row_grad.has_rows) else None
        if dense is None and sparse is None:
            return loss                       # no gradient: torch leaves the parameter alone
        t = self.t + 1
        if t >= self.hist.shape[0]:
            grown = torch.zeros(2 * self.hist.shape[0], 4, device=self.hist.device, dtype=torch.float32)
            grown[: self.hist.shape[0]] = self.hist
            self.hist = grown
        scalars = self._step_scalars(t)
        if dense is not None:
            if dense.is_sparse:
                raise ValueError("BankAdamW takes a dense or row-sparse (RowSparseBankGrad) bank gradient")
            g = dense.float().contiguous()
            if sparse is not None:            # both kinds this step: fold the rows into the dense gradient
                g = g + sparse.to_dense()
            self._run(g, None, None, 0, t, scalars)
        else:
            lst, n = sparse.touched()
            self._run(sparse.acc, lst, n, sparse.max_touched, t, scalars, grad_scale=sparse.scale)
        self.t = t
        self.state[self.bank]["step"] = torch.tensor(float(t))
        return loss

    def zero_grad(self, set_to_none: bool = True) -> None:
        super().zero_grad(set_to_none=set_to_none)
        if self.row_grad is not None:
            self.row_grad.zero_()

    # ------------------------------------------------------------------ state
    def state_dict(self):
        """``torch.optim.AdamW``'s format for the bank (after a flush), so it loads into AdamW."""
        self.flush()
        st = {"step": torch.tensor(float(self.t)), "exp_avg": self.exp_avg, "exp_avg_sq": self.exp_avg_sq}
        groups = [{k: v for k, v in self.param_groups[0].items() if k != "params"}]
        groups[0].update(params=[0], amsgrad=False, maximize=False, foreach=None, capturable=False,
                         differentiable=False, fused=None)
        return {"state": {0: st}, "param_groups": groups}

    def load_state_dict(self, state_dict) -> None:
        st = state_dict["state"].get(0)
        grp = state_dict["param_groups"][0]
        for k in ("lr", "betas", "eps", "weight_decay"):
            if k in grp:
                self.param_groups[0][k] = tuple(grp[k]) if k == "betas" else grp[k]
        if st is None:
            self.t = 0
            self.exp_avg.zero_()
            self.exp_avg_sq.zero_()
        else:
            self.t = int(float(st["step"]))
            self.exp_avg.copy_(st["exp_avg"])
            self.exp_avg_sq.copy_(st["exp_avg_sq"])
        self.tags.fill_(self.t)
        if self.t >= self.hist.shape[0]:
            self.hist = torch.zeros(2 * self.t + 2, 4, device=self.hist.device, dtype=torch.float32)
        if self.mirror is not None:
            self.mirror.copy_(self.bank.detach())
        self.state[self.bank]["step"] = torch.tensor(float(self.t))


def clip_grad_norm_(parameters, max_norm: float, norm_type: float = 2.0) -> torch.Tensor:
    """``torch.nn.utils.clip_grad_norm_`` (trainer.py:876-882) for parameters whose gradient may
    be row-sparse (a ``RowSparseBankGrad`` attached to the bank): the total 2-norm counts those
    rows, dense gradients are scaled in place and the bank's coefficient is handed to its
    optimizer step.  Returns the total norm (device tensor)."""
    if float(norm_type) != 2.0:
        raise NotImplementedError("clip_grad_norm_ with row-sparse gradients supports norm_type=2")
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    params = list(parameters)
    grads = [p.grad for p in params if p.grad is not None]
    sinks = []
    for p in params:
        s = getattr(p, "_moc_row_grad", None)
        if s is not None and s.has_rows and s not in sinks:
            sinks.append(s)
    norms = [torch.linalg.vector_norm(g.detach(), 2.0).float() for g in grads]
    norms += [s.sqnorm().sqrt().reshape(()) for s in sinks]
    if not norms:
        return torch.tensor(0.0)
    total = torch.linalg.vector_norm(torch.stack(norms), 2.0)
    coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    if grads:
        torch._foreach_mul_(grads, coef.to(grads[0].device))
    for s in sinks:
        s.scale = coef.reshape(1).float().contiguous() if s.scale is None else (s.scale * coef).reshape(1)
    return total
