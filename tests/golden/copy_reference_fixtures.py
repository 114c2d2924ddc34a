"""Copies the reference's own frozen test fixtures (data only: inputs and expected
outputs) into tests/golden/ and records their provenance in MANIFEST.txt. Run in the
build container, where the reference is mounted read-only at /root/reference:

    python tests/golden/copy_reference_fixtures.py

- equivalence_fixtures.npz + equivalence_torch_reference.json:
  param_decomp/param_decomp/tests/targets/equivalence/{fixtures.npz,torch_reference.json}
  (a tiny GLU-MLP suffix with zeroed attention, pre-drawn masks and PPGD sources; the
  frozen torch-era loss goldens).
- simple_mlp_tiny_fixture.npz:
  param_decomp/param_decomp/tests/targets/simple_mlp_equivalence/tiny_fixture.npz
  (a 3-layer LlamaSimpleMLP state dict, token ids and the torch fp32 logits).
- stacked_sources.npz: the `src::*` arrays of
  param_decomp/param_decomp/tests/targets/stacked_parity/stacked_fixtures.npz (the
  persistent sources its generator drew with jax.random from PRNGKey(3): one fp32 uniform
  draw of [1, 16, 9] per site under split(PRNGKey(3), 9), site order as stored).
- stacked_forward.npz: the forward pins of the same file (a residual-fed tiny GLU Llama,
  layers 3-7, with the MLP sites of layers 3-5 decomposed): the frozen target and V/U
  (`tgt::*`, `vu::*`), the input `resid`, the fixed masks, delta masks and layer-3 routes
  (`mask::*`, `delta_mask::*`, `route0::*`) and the fp32 logits `out::clean`,
  `out::masked_all` and `out::masked_subset` (the route arm).
"""

import hashlib
import os
import shutil

REF = "/root/reference/param_decomp/param_decomp/tests/targets"
HERE = os.path.dirname(os.path.abspath(__file__))
FILES = [
    ("equivalence/fixtures.npz", "equivalence_fixtures.npz"),
    ("equivalence/torch_reference.json", "equivalence_torch_reference.json"),
    ("simple_mlp_equivalence/tiny_fixture.npz", "simple_mlp_tiny_fixture.npz"),
]


SUBSETS = [  # (reference file, destination, key prefixes kept)
    ("stacked_parity/stacked_fixtures.npz", "stacked_sources.npz", ("src::",)),
    ("stacked_parity/stacked_fixtures.npz", "stacked_forward.npz",
     ("tgt::", "vu::", "mask::", "delta_mask::", "route0::", "resid", "out::clean", "out::masked_", "_scalar_")),
]


def main() -> None:
    import numpy as np

    lines = []
    for src, dst in FILES:
        shutil.copyfile(os.path.join(REF, src), os.path.join(HERE, dst))
        digest = hashlib.sha256(open(os.path.join(HERE, dst), "rb").read()).hexdigest()
        lines.append(f"{dst}  sha256={digest}  from param_decomp/param_decomp/tests/targets/{src}")
    for src, dst, prefixes in SUBSETS:
        z = np.load(os.path.join(REF, src), allow_pickle=False)
        keep = {k: z[k] for k in z.keys() if k.startswith(prefixes)}
        np.savez(os.path.join(HERE, dst), **keep)
        digest = hashlib.sha256(open(os.path.join(REF, src), "rb").read()).hexdigest()
        pat = ", ".join(p + "*" for p in prefixes)
        lines.append(f"{dst}  arrays {pat} ({len(keep)}) of param_decomp/param_decomp/tests/targets/{src} "
                     f"(sha256={digest})")
    with open(os.path.join(HERE, "MANIFEST.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


if __name__ == "__main__":
    main()
