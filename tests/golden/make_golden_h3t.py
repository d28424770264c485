"""Write tests/golden/vectors/h3t_tiny_quant.h3t with the REFERENCE's own .h3t writer.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden_h3t.py [--reference /root/reference]

What it pins: the exact bytes of the container (header JSON and its formatting, metadata keys and their order,
the canonical tensor order, 256-byte tensor and 4 KiB block alignment, padding entries) for a tiny 2-block W4A8
checkpoint from h3t_inputs.state_dict(), which no closed form covers.  The file is data: tests compare this
build's writer output with it byte for byte and read it with this build's reader.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import h3t_inputs as hi  # noqa: E402

OUT = os.path.join(HERE, "vectors", "h3t_tiny_quant.h3t")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    a = ap.parse_args()
    sys.path.insert(0, a.reference)
    from h3turbo.h3.config import H3Config
    from h3turbo.h3.writer import write_h3t

    sd = hi.state_dict(quant=True, seed=0)
    rep = write_h3t(OUT, H3Config(**hi.TINY), sd, source_name="tiny", source_size=123)
    data = open(OUT, "rb").read()
    print(json.dumps({"file": os.path.relpath(OUT, HERE), "sha256": hashlib.sha256(data).hexdigest(), **rep}))


if __name__ == "__main__":
    main()
