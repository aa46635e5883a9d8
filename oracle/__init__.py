"""CPU oracle for the Muon / Newton–Schulz hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's arithmetic for the path that
``pan2_amd`` runs on the GPU. It is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import it, and nothing in ``pan2_amd`` does.

Modules:
  bf16          round-to-nearest-even fp32 -> bf16 in numpy
  muon_ref      momentum, adjust_lr, param step, standard and gram-form NS,
                full Muon step (each function cites the reference line it follows)
  cpu_baseline  times the reference's CPU path (stock torch.optim.Muon with a
                float lr, as pan/optim/muon.py:126-154 builds it)

Pinning status (what checks each function; see tests/test_oracle_*.py):
  round_bf16            torch's own fp32->bf16 cast on ties, NaN, Inf, subnormals
  adjust_lr_ratio       torch.optim._muon._adjust_lr over every mode x shape class
  momentum_nesterov     torch's lerp form (<= 1 ulp) and brute force on scalars
  step_param            brute force on scalars; torch's mul_/add_ form
  ns_standard fp64      closed form U diag(p^k(s/|s|)) V^T on constructed SVDs,
                        transpose / scale / zero / NaN invariants
  ns_standard bf16      torch's stock _zeropower_via_newtonschulz (CPU) and the
                        committed golden vectors
  ns_gram               equals ns_standard in exact arithmetic (fp64, 1e-10)
  muon_step             stock torch.optim.Muon (CPU) step and golden vectors
Each check is also run against planted mistakes (tests/test_oracle_mutants.py)
so a dropped term, a flipped sign or a transposed operand fails it.
"""
