"""Planted mistakes in the CPU oracle must fail the checks that pin it.

Each case rewrites one line of a copy of oracle/muon_ref.py (or oracle/bf16.py)
in memory, loads the copy as a module and runs the pinning checks of
tests/pins.py against it; at least one check has to fail. The oracle files on
disk are never changed.
"""
import inspect
import types

import pytest

import oracle.bf16
import oracle.muon_ref
from tests import pins


def _mutant(module, old: str, new: str, name: str):
    src = inspect.getsource(module)
    assert src.count(old) >= 1, f"mutation anchor not found in {module.__name__}: {old!r}"
    src = src.replace(old, new, 1)
    mod = types.ModuleType(f"oracle._mutant_{name}")
    mod.__package__ = "oracle"
    mod.__file__ = module.__file__
    exec(compile(src, f"<mutant {name}>", "exec"), mod.__dict__)
    return mod


MUON_CHECKS = (pins.check_adjust_lr, pins.check_momentum, pins.check_step, pins.check_ns_closed_form,
               pins.check_ns_invariants, pins.check_ns_bf16_vs_torch, pins.check_ns_gram,
               pins.check_muon_step_vs_torch)

# (name, old text, new text): each is a plausible slip in the restatement
MUON_MUTANTS = [
    ("adjust_min_for_max", "0.2 * math.sqrt(max(A, B))", "0.2 * math.sqrt(min(A, B))"),
    ("adjust_ratio_inverted", "math.sqrt(max(1, A / B))", "math.sqrt(max(1, B / A))"),
    ("momentum_weights_swapped", "nb = (mu * b).astype(np.float32) + (omu * g)",
     "nb = (omu * b).astype(np.float32) + (mu * g)"),
    ("nesterov_uses_old_buffer", "(mu * nb).astype(np.float32)).astype(np.float32)",
     "(mu * b).astype(np.float32)).astype(np.float32)"),
    ("step_sign_flipped", "(u * neg).astype(np.float32)", "(u * -neg).astype(np.float32)"),
    ("wd_uses_adjusted_lr", "f32(1.0 - lr * weight_decay)", "f32(1.0 - lr * ratio * weight_decay)"),
    ("ns_dropped_b_term", "B = rnd(dt(c) * (A @ A) + dt(b) * A)", "B = rnd(dt(c) * (A @ A))"),
    ("ns_sign_of_c", "B = rnd(dt(c) * (A @ A) + dt(b) * A)", "B = rnd(-dt(c) * (A @ A) + dt(b) * A)"),
    ("ns_coeff_order", "for a, b, c in coeffs:\n        A = rnd(X @ X.T)", "for a, c, b in coeffs:\n        A = rnd(X @ X.T)"),
    ("ns_squared_norm", "X = rnd((X / nrm).astype(dt))\n    for a, b, c in coeffs:\n        A",
     "X = rnd((X / (nrm * nrm)).astype(dt))\n    for a, b, c in coeffs:\n        A"),
    ("ns_missing_iteration", "coeffs = _coeff_list(ns_coefficients, ns_steps)\n    X = rnd(G.astype(dt))\n    tall",
     "coeffs = _coeff_list(ns_coefficients, ns_steps)[1:]\n    X = rnd(G.astype(dt))\n    tall"),
    ("ns_no_transpose_back", "    if tall:\n        X = np.ascontiguousarray(X.T)\n    return X\n\n\ndef ns_gram",
     "    return X\n\n\ndef ns_gram"),
    ("ns_update_wrong_row_index", "X = rnd(dt(a) * X + B @ X)", "X = rnd(dt(a) * X + B @ X[::-1])"),
    ("ns_gram_transposed_operand", "A = rnd(X @ X.T)\n        B = rnd", "A = rnd(X.T @ X)\n        B = rnd"),
    ("gram_rz_wrong_coeff", "RZ = rnd(R @ Z + dt(a) * R)", "RZ = rnd(R @ Z + dt(b) * R)"),
    ("gram_no_regram_at_reset", "X = rnd(Q @ X)\n            R = rnd(X @ X.T)", "X = rnd(Q @ X)"),
    ("quintic_power_dropped_cubic", "x = a * x + b * x ** 3 + c * x ** 5", "x = a * x + c * x ** 5"),
]


@pytest.mark.parametrize("name,old,new", MUON_MUTANTS, ids=[m[0] for m in MUON_MUTANTS])
def test_planted_mistake_is_caught(name, old, new):
    mod = _mutant(oracle.muon_ref, old, new, name)
    failed = []
    for check in MUON_CHECKS:
        try:
            check(mod)
        except (AssertionError, ValueError):
            failed.append(check.__name__)
    assert failed, f"no pinning check caught the planted mistake {name!r}"


BF16_MUTANTS = [
    ("ties_away_from_zero", "(u + np.uint64(0x7FFF) + lsb)", "(u + np.uint64(0x8000))"),
    ("truncate", "(u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)", "u >> np.uint64(16)"),
    ("nan_not_quieted", "| np.uint64(0x40)", "| np.uint64(0x0)"),
]


@pytest.mark.parametrize("name,old,new", BF16_MUTANTS, ids=[m[0] for m in BF16_MUTANTS])
def test_planted_bf16_mistake_is_caught(name, old, new):
    mod = _mutant(oracle.bf16, old, new, name)
    with pytest.raises(AssertionError):
        pins.check_round_bf16(mod)


def test_unmutated_copy_passes_every_check():
    """The copy machinery itself changes nothing."""
    mod = _mutant(oracle.muon_ref, "EPS = 1e-7", "EPS = 1e-7", "identity")
    for check in MUON_CHECKS:
        check(mod)
    pins.check_round_bf16(_mutant(oracle.bf16, "import numpy as np", "import numpy as np", "identity_bf16"))


ADAM_CHECKS = (pins.check_adam_vs_torch, pins.check_adam_closed_form)

ADAM_MUTANTS = [
    ("betas_swapped", "m = lerp(m, gr, 1 - beta1)", "m = lerp(m, gr, 1 - beta2)"),
    ("no_first_bias_correction", "step_size = lr / bc1", "step_size = lr"),
    ("second_correction_not_rooted", "bc2_sqrt = bc2 ** 0.5", "bc2_sqrt = bc2"),
    ("step_not_incremented", "step = float(f32(step) + f32(1))", "step = float(f32(step) + f32(2))"),
    ("adamw_decay_coupled", "p = p * f32(1 - lr * weight_decay)", "gr = gr + f32(weight_decay) * p"),
    ("eps_inside_sqrt", "np.sqrt(vh) / f32(bc2_sqrt) + f32(eps)", "np.sqrt(vh + f32(eps)) / f32(bc2_sqrt)"),
    ("update_sign", "p = p + f32(-step_size)", "p = p + f32(step_size)"),
    ("lerp_upper_branch", "return end - (end - start) * (f32(1) - w)", "return end - (end - start) * w"),
    ("maximize_ignored", "gr = -g if maximize else g", "gr = g"),
    ("amsgrad_uses_current_v", "        vh = vmax\n", "        vh = v\n"),
]


@pytest.mark.parametrize("name,old,new", ADAM_MUTANTS, ids=[m[0] for m in ADAM_MUTANTS])
def test_planted_adam_mistake_is_caught(name, old, new):
    import oracle.adamw_ref

    mod = _mutant(oracle.adamw_ref, old, new, name)
    failed = []
    for check in ADAM_CHECKS:
        try:
            check(mod)
        except (AssertionError, ValueError, FloatingPointError):
            failed.append(check.__name__)
    assert failed, f"no pinning check caught the planted mistake {name!r}"
