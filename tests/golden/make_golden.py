"""Writes tests/golden/torch_muon_cpu.npz: golden vectors of the reference's CPU path.

The reference's CPU path is torch's stock Muon (pan/optim/muon.py:126 leaves
it unpatched for a float lr; TORCH/optim/_muon.py:31-70,285-318). This script
runs that stock code on the CPU (PyTorch only; nothing from the reference is
imported) on small seeded inputs and stores inputs and outputs:

  ns/<case>/in         fp32 input G
  ns/<case>/out_bf16   uint16 bf16 bits of _zeropower_via_newtonschulz(G)
  step/<case>/{p0,g,b0,p1,b1,lr,wd,adjust}   one Muon.step() with a float lr

Run from the repo root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
COEFFS = (3.4445, -4.7750, 2.0315)

NS_CASES = {
    "wide_32x128": (32, 128, 101),
    "tall_128x32": (128, 32, 102),
    "square_64": (64, 64, 103),
    "ragged_48x80": (48, 80, 104),
    "ragged_tall_72x40": (72, 40, 105),
}
STEP_CASES = {
    "wide_48x96_none": (48, 96, None, 201),
    "tall_96x48_rms": (96, 48, "match_rms_adamw", 202),
}


def main() -> int:
    import torch.optim._muon as tm

    zeropower = tm._zeropower_via_newtonschulz
    out = {}
    for name, (m, n, seed) in NS_CASES.items():
        g = torch.Generator("cpu").manual_seed(seed)
        G = torch.randn(m, n, generator=g)
        O = zeropower(G.clone(), COEFFS, 5, 1e-7)
        out[f"ns/{name}/in"] = G.numpy()
        out[f"ns/{name}/out_bf16"] = O.view(torch.int16).numpy().view(np.uint16)
    for name, (m, n, adjust, seed) in STEP_CASES.items():
        g = torch.Generator("cpu").manual_seed(seed)
        p0 = torch.randn(m, n, generator=g) * 0.02
        gr = torch.randn(m, n, generator=g) * 1e-3
        b0 = torch.randn(m, n, generator=g) * 1e-3
        p = torch.nn.Parameter(p0.clone())
        p.grad = gr.clone()
        opt = torch.optim.Muon([p], lr=0.02, weight_decay=0.01, momentum=0.95, adjust_lr_fn=adjust)
        opt.state[p]["momentum_buffer"] = b0.clone()
        opt.step()
        for k, v in (("p0", p0), ("g", gr), ("b0", b0), ("p1", p.detach()), ("b1", opt.state[p]["momentum_buffer"])):
            out[f"step/{name}/{k}"] = v.numpy().astype(np.float32)
        out[f"step/{name}/lr"] = np.float64(0.02)
        out[f"step/{name}/wd"] = np.float64(0.01)
        out[f"step/{name}/adjust"] = np.str_(str(adjust))
    out["meta/torch_version"] = np.str_(torch.__version__)
    path = os.path.join(HERE, "torch_muon_cpu.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, torch {torch.__version__})")
    return 0


if __name__ == "__main__":
    sys.exit(main())
