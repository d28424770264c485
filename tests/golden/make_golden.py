"""Write the golden vectors under tests/golden/ by running the REFERENCE's own qlinear (torch CPU backend).

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden.py [--reference /root/reference]

What it pins: the full bit-exact chain of the reference's quantize_activation / decode_int8_grid / _int8_mm /
linear on Gaussian + outlier inputs (the fp64->fp32->bf16 rounding chain, torch's bf16 division and the
int32*fp32 promotion), which no closed form covers.  Inputs come from tests/golden/inputs.py (seeded); the
fixtures store the input hashes so a test can prove it regenerated the same inputs.  Large outputs are stored
as SHA-256 plus a slice of leading rows; small cases are stored whole.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

OUT = os.path.join(HERE, "vectors")


def to_t_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def weight(ql_types, q, s_rel, s_kind, s_ch, cb, group, convrot):
    if s_kind == "fp8":
        s = torch.from_numpy(s_rel.copy()).view(torch.float8_e4m3fn)
    elif s_kind == "f16":
        s = torch.from_numpy(s_rel.view(np.int16).copy()).view(torch.float16)
    else:
        s = torch.from_numpy(s_rel.astype(np.float32))
    return ql_types.W4A8Weight(torch.from_numpy(q.copy()), s, torch.from_numpy(s_ch.copy()), torch.from_numpy(cb.copy()),
                               group_size=group, convrot=convrot)


def out_bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    from h3turbo.h3 import qlinear as ql  # the reference, in this container only
    from h3turbo.h3 import types as ql_types

    torch.set_num_threads(os.cpu_count() or 1)
    os.makedirs(OUT, exist_ok=True)
    index = {}

    def save(name, meta, arrays):
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **arrays)
        index[name] = meta
        print(f"  wrote {name}: {sorted(arrays)}", flush=True)

    dt_of = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}

    # ---------------------------------------------------------------- small cases, stored whole
    print("small cases", flush=True)
    for (m, k, n, group, convrot, s_kind, x_dt, mode, with_bias, seed) in [
        (1, 512, 40, 16, 256, "fp8", "bf16", "ck", False, 1),
        (7, 512, 40, 16, 256, "fp8", "bf16", "ck", True, 2),
        (33, 512, 40, 16, 256, "fp8", "bf16", "eager", False, 3),
        (17, 512, 40, 16, 256, "fp8", "f32", "ck", False, 4),
        (17, 512, 40, 16, 256, "fp8", "f16", "ck", True, 5),
        (64, 1024, 48, 128, 256, "f16", "bf16", "ck", False, 6),
        (5, 256, 24, 4, 64, "fp8", "bf16", "ck", False, 7),
        (9, 128, 16, 32, 16, "fp8", "bf16", "eager", True, 8),
        (300, 256, 72, 16, 256, "fp8", "bf16", "ck", True, 9),
    ]:
        xb = gi.activations(m, k, seed=seed)
        x = to_t_bf16(xb).to(dt_of[x_dt])
        if s_kind == "fp8":
            q, s_rel, s_ch, cb = gi.weight_fp8_g16(n, k, seed=seed, group=group)
        else:
            q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=seed, group=group, convrot=convrot)
        w = weight(ql_types, q, s_rel, s_kind, s_ch, cb, group, convrot)
        b = gi.bias(n, seed) if with_bias else None
        xq, xs = ql.quantize_activation(x, size=convrot, quant_mode=mode)
        w8 = ql.decode_int8_grid(w)
        acc = ql._int8_mm(xq, w8)
        out = ql.linear(x, w, None if b is None else torch.from_numpy(b), backend="torch", quant_mode=mode)
        name = f"small_m{m}_k{k}_n{n}_g{group}_r{convrot}_{s_kind}_{x_dt}_{mode}{'_bias' if with_bias else ''}"
        x_store = x.float().numpy() if x_dt == "f32" else out_bits(x)
        arrays = dict(x=x_store, q=q, s_rel=s_rel, s_ch=s_ch, cb=cb, xq=xq.numpy(), xs=xs.numpy(), w8=w8.numpy(),
                      acc=acc.numpy(), out=out_bits(out))
        if n * k > 32768:
            del arrays["w8"]  # decode is pinned by its own element-loop checks; keep the fixture small
        if b is not None:
            arrays["bias"] = b
        save(name, dict(m=m, k=k, n=n, group=group, convrot=convrot, s_kind=s_kind, x_dtype=x_dt, mode=mode,
                        bias=with_bias, seed=seed, kind="small"), arrays)

    # swiglu (fc2-style input), stored whole
    m, k, n = 9, 512, 40
    g = torch.Generator().manual_seed(18)
    h = torch.randn(m, 2 * k, generator=g).to(torch.bfloat16)
    q, s_rel, s_ch, cb = gi.weight_fp8_g16(n, k, seed=11)
    w = weight(ql_types, q, s_rel, "fp8", s_ch, cb, 16, 256)
    out = ql.linear(h, w, backend="torch", input_act="swiglu")
    act = ql._swiglu(h)
    save("swiglu_m9_k512_n40", dict(m=m, k=k, n=n, group=16, convrot=256, s_kind="fp8", x_dtype="bf16", mode="ck",
                                    kind="swiglu"),
         dict(h=out_bits(h), act=out_bits(act), q=q, s_rel=s_rel, s_ch=s_ch, cb=cb, out=out_bits(out)))

    # ---------------------------------------------------------------- config 1 (hash + leading rows)
    print("config 1", flush=True)
    for s_kind in ("f16", "fp8"):
        m, k, n = 256, 1024, 1024
        xb = gi.activations(m, k, seed=0)
        if s_kind == "f16":
            q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=0)
            group = 128
        else:
            q, s_rel, s_ch, cb = gi.weight_fp8_g16(n, k, seed=0)
            group = 16
        x = to_t_bf16(xb)
        w = weight(ql_types, q, s_rel, s_kind, s_ch, cb, group, 256)
        t0 = time.perf_counter()
        xq, xs = ql.quantize_activation(x)
        w8 = ql.decode_int8_grid(w)
        acc = ql._int8_mm(xq, w8)
        out = ql.linear(x, w, backend="torch")
        out_e = ql.linear(x, w, backend="torch", quant_mode="eager")
        print(f"  reference c1 ({s_kind}) took {time.perf_counter() - t0:.2f}s", flush=True)
        meta = dict(m=m, k=k, n=n, group=group, convrot=256, s_kind=s_kind, x_dtype="bf16", kind="c1",
                    sha_inputs=gi.sha(xb, q, s_rel, s_ch, cb), sha_xq=gi.sha(xq.numpy()), sha_xs=gi.sha(xs.numpy()),
                    sha_w8=gi.sha(w8.numpy()), sha_acc=gi.sha(acc.numpy()), sha_out=gi.sha(out_bits(out)),
                    sha_out_eager=gi.sha(out_bits(out_e)))
        save(f"c1_{s_kind}", meta, dict(xq=xq.numpy()[:16], xs=xs.numpy(), acc=acc.numpy()[:8], out=out_bits(out)[:16],
                                        out_eager=out_bits(out_e)[:8]))

    # ---------------------------------------------------------------- config 2 (rotation + quant, hashes)
    print("config 2", flush=True)
    m, k = 12090, 5120
    xb = gi.activations(m, k, seed=0)
    t0 = time.perf_counter()
    xq, xs = ql.quantize_activation(to_t_bf16(xb))
    print(f"  reference c2 took {time.perf_counter() - t0:.2f}s", flush=True)
    save("c2", dict(m=m, k=k, convrot=256, x_dtype="bf16", kind="c2", sha_inputs=gi.sha(xb), sha_xq=gi.sha(xq.numpy()),
                    sha_xs=gi.sha(xs.numpy())),
         dict(xq=xq.numpy()[:4], xs=xs.numpy()))

    # ---------------------------------------------------------------- config 3 at M=512 (hashes)
    print("config 3 (M=512)", flush=True)
    for k, n in ((5120, 5120), (5120, 15360), (5120, 13824), (13824, 5120)):
        m = 512
        xb = gi.activations(m, k, seed=0)
        q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=0)
        w = weight(ql_types, q, s_rel, "f16", s_ch, cb, 128, 256)
        x = to_t_bf16(xb)
        t0 = time.perf_counter()
        xq, xs = ql.quantize_activation(x)
        acc = ql._int8_mm(xq, ql.decode_int8_grid(w))
        out = ql.linear(x, w, backend="torch")
        print(f"  reference c3 k={k} n={n} took {time.perf_counter() - t0:.2f}s", flush=True)
        save(f"c3_m{m}_k{k}_n{n}", dict(m=m, k=k, n=n, group=128, convrot=256, s_kind="f16", x_dtype="bf16", kind="c3",
                                         sha_inputs=gi.sha(xb, q, s_rel, s_ch, cb), sha_xq=gi.sha(xq.numpy()),
                                         sha_xs=gi.sha(xs.numpy()), sha_acc=gi.sha(acc.numpy()), sha_out=gi.sha(out_bits(out))),
             dict(out=out_bits(out)[:2], acc=acc.numpy()[:1]))

    meta = dict(generator="tests/golden/make_golden.py", torch=torch.__version__, numpy=np.__version__,
                reference="h3turbo.h3.qlinear (torch backend, CPU)", cases=index)
    with open(os.path.join(OUT, "index.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("done", flush=True)


if __name__ == "__main__":
    main()
