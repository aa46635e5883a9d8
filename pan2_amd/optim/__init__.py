"""Drop-in for PAN 2's pan/optim package, running Muon on libpanmuon (gfx950).

Like the reference's pan/optim (a namespace package with no re-exports), import
from the submodules: ``pan2_amd.optim.muon`` (build_native_muon_optimizers,
split_params_for_native_muon), ``pan2_amd.optim.patch_muon`` (patch_muon,
newton_schulz), ``pan2_amd.optim.patch_lr_scheduler`` and
``pan2_amd.optim.kernels`` (muon_momentum_nesterov, step_param).
"""
