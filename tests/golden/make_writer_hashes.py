"""Extract the VQ-tensor known answers from the reference's writer goldens.

The reference pins what its writers produce as sha256[:16] of each tensor's
bytes (tests/test_writer_contracts.py:195-216, goldens under
tests/golden/writers/). Three of those goldens cover this path:

  pack.json / pack_straddle.json   packed uint32 codes [2,128,4] (K16 -> 4
                                   bits, d4) plus the untouched codebooks and
                                   scales
  sz_pack.json                     unpacked uint8 codes [2,128,32] and the
                                   skipzero tensors sz_codes / sz_scales /
                                   sz_rowmask / sz_shape of the one module
                                   with dead rows

This script copies only those hashes, shapes and dtypes (data, not source)
into writer_hashes.json next to it. It reads the reference checkout, so it
runs in the build container only; the JSON it writes is what the tests use.

    python tests/golden/make_writer_hashes.py /root/reference
"""
from __future__ import annotations

import json
import pathlib
import sys

HERE = pathlib.Path(__file__).resolve().parent
SUFFIXES = (".codes", ".codebook", ".vq_scales", ".sz_codes", ".sz_scales",
            ".sz_rowmask", ".sz_shape")


def main(ref_root: str) -> None:
    src = pathlib.Path(ref_root) / "tests" / "golden" / "writers"
    out = {}
    for name in ("pack", "pack_straddle", "sz_pack"):
        gold = json.loads((src / f"{name}.json").read_text())
        keep = {}
        for k, v in sorted(gold["tensors"].items()):
            if ".mlp.switch_mlp." in k and k.endswith(SUFFIXES):
                keep[k] = {"dtype": v["dtype"], "shape": v["shape"], "sha": v["sha"]}
        mods = gold["config"].get("vq_modules", {})
        out[name] = {
            "tensors": keep,
            "vq_modules": {k: mods[k] for k in sorted(mods)},
            "vq_skipzero": gold["config"].get("vq_skipzero", {}).get("modules"),
        }
    (HERE / "writer_hashes.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {HERE / 'writer_hashes.json'}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
