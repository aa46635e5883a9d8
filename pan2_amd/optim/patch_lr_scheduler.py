"""Host-side ``LambdaLR.get_last_lr()`` for tensor learning rates.

Drop-in for pan/optim/patch_lr_scheduler.py: with a tensor lr, LambdaLR keeps
``base_lrs`` as device tensors, so reading the last lr would sync the device.
After :func:`patch_lr_scheduler`, ``get_last_lr()`` evaluates
``base_lr * lr_lambda(last_epoch)`` on the host from a one-time host copy of
the base values (re-read only when ``base_lrs`` is replaced). The values the
scheduler writes into the optimizer are unchanged.
"""
from __future__ import annotations

from weakref import WeakKeyDictionary

from torch.optim.lr_scheduler import LambdaLR

# scheduler -> (the base_lrs list object, its values as python floats)
_host_copy: "WeakKeyDictionary[LambdaLR, tuple[list, list[float]]]" = WeakKeyDictionary()


def _host_base_lrs(sched: LambdaLR) -> list[float]:
    entry = _host_copy.get(sched)
    if entry is None or entry[0] is not sched.base_lrs:
        entry = (sched.base_lrs, [float(v) for v in sched.base_lrs])
        _host_copy[sched] = entry
    return entry[1]


def _get_last_lr_host(self: LambdaLR) -> list[float]:
    bases = _host_base_lrs(self)
    if len(bases) != len(self.lr_lambdas):
        raise ValueError("base_lrs and lr_lambdas differ in length")
    return [base * fn(self.last_epoch) for base, fn in zip(bases, self.lr_lambdas)]


def patch_lr_scheduler() -> None:
    LambdaLR.get_last_lr = _get_last_lr_host
