"""Host-side ``LambdaLR.get_last_lr()`` for tensor learning rates.

Drop-in for the ``patch_lr_scheduler`` of pan/optim/patch_lr_scheduler.py:38-39,
which replaces ``LambdaLR.get_last_lr``. With a tensor lr, LambdaLR keeps
``base_lrs`` as device tensors, and torch's ``get_last_lr()`` hands back
device values, so every log line that reads them waits for the device.

Here the base learning rates are read to the host when a LambdaLR is
constructed and when ``load_state_dict`` replaces its state (both wrapped by
:func:`patch_lr_scheduler`), and again whenever ``get_last_lr()`` finds that
``base_lrs`` is no longer the list object they were read from (a direct
assignment, or a subclass whose ``load_state_dict`` bypasses the wrapper); a
scheduler built before the patch is read on its first ``get_last_lr()``.
``get_last_lr()`` evaluates ``base * lr_lambda(last_epoch)`` from those host
floats; its only device reads are those re-captures. The host copies live in
a side table keyed by the scheduler (not in its ``__dict__``, which
``state_dict()`` serialises). The learning rates the scheduler writes into
the optimizer are untouched. Changing an element of ``base_lrs`` in place is
not tracked (the list object stays the same).
"""
from __future__ import annotations

import functools
from weakref import WeakKeyDictionary

from torch.optim.lr_scheduler import LambdaLR

# scheduler -> (the base_lrs list object that was read, its values as host floats)
_bases: "WeakKeyDictionary[LambdaLR, tuple[list, tuple[float, ...]]]" = WeakKeyDictionary()


def _capture(sched: LambdaLR) -> tuple[float, ...]:
    """Reads the scheduler's base learning rates to the host (one device read each)."""
    src = sched.base_lrs
    vals = tuple(float(b) for b in src)
    if len(vals) != len(sched.lr_lambdas):
        raise ValueError(f"{len(vals)} base learning rates for {len(sched.lr_lambdas)} lr_lambdas")
    _bases[sched] = (src, vals)
    return vals


def _get_last_lr(self: LambdaLR) -> list[float]:
    entry = _bases.get(self)
    # an identity test: no device read unless base_lrs was replaced
    vals = entry[1] if entry is not None and entry[0] is self.base_lrs else _capture(self)
    epoch = self.last_epoch
    return [b * fn(epoch) for b, fn in zip(vals, self.lr_lambdas)]


def _wrap_once(name: str, after):
    """Wraps LambdaLR.<name> so that after(self) runs once the original returns."""
    orig = getattr(LambdaLR, name)
    if getattr(orig, "_pan2_host_lr", False):
        return

    @functools.wraps(orig)
    def wrapped(self, *args, **kwargs):
        out = orig(self, *args, **kwargs)
        after(self)
        return out

    wrapped._pan2_host_lr = True
    setattr(LambdaLR, name, wrapped)


def patch_lr_scheduler() -> None:
    _wrap_once("__init__", _capture)
    _wrap_once("load_state_dict", _capture)
    LambdaLR.get_last_lr = _get_last_lr
