"""Write tests/golden/reference_vectors.npz from the reference's own CPU code.

Runs oracle/_ref/libref.so (miniTensor's matmul / conv2d / Linear CPU path
and conv2d's autograd backward, compiled from its headers by oracle/Makefile)
on small seeded inputs and stores inputs and outputs as plain arrays
(np.savez, no pickles), plus the same arrays as a raw binary for the C++
host-layer tests, so the oracle, the host layer's CPU device and the GPU path
can be checked against the reference where the reference tree is not
available.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "reference_vectors.npz"


def write_bin(arrays: dict, path: Path) -> None:
    """The same arrays in a raw form a C++ test reads without numpy:
    b"MTGOLD01", count (u32), then per array: name length (u32), name,
    ndim (u32), dims (u64 each), the float32 data (little-endian)."""
    with open(path, "wb") as f:
        f.write(b"MTGOLD01")
        f.write(np.uint32(len(arrays)).tobytes())
        for name in sorted(arrays):
            a = np.ascontiguousarray(arrays[name], dtype=np.float32)
            nb = name.encode()
            f.write(np.uint32(len(nb)).tobytes() + nb)
            f.write(np.uint32(a.ndim).tobytes())
            f.write(np.asarray(a.shape, dtype=np.uint64).tobytes())
            f.write(a.astype("<f4").tobytes())
    print(f"wrote {path} ({path.stat().st_size} bytes)")


def main() -> None:
    oracle.build()
    r = oracle.ref()
    fp = oracle._fp
    v = {}

    # 1. 3x5 · 5x4 with offset views: A is rows 2..4 of a [5,5] storage, B is
    #    a [5,4] view at offset 3 of a flat buffer.
    a_store = oracle.uniform((25,), 42)
    b_store = oracle.uniform((3 + 20,), 43)
    c = np.empty((3, 4), np.float32)
    r.ref_matmul_view_f32(fp(a_store), 25, 10, 5, 1, fp(b_store), 23, 3, 4, 1, 3, 5, 4, fp(c))
    v["offset_a_store"], v["offset_b_store"], v["offset_c"] = a_store, b_store, c

    # 2. 33x47 · (29x47)ᵀ: B passed as a transpose view (strides (1,47)).
    a = oracle.uniform((33, 47), 44)
    bt = oracle.uniform((29, 47), 45)
    c = np.empty((33, 29), np.float32)
    r.ref_matmul_view_f32(fp(a), a.size, 0, 47, 1, fp(bt), bt.size, 0, 1, 47, 33, 47, 29, fp(c))
    v["bT_a"], v["bT_bt"], v["bT_c"] = a, bt, c

    # 3. expand view: a [1,40] row broadcast to [17,40] (stride 0) times [40,23]
    row = oracle.normal((40,), 46)
    b = oracle.normal((40, 23), 47)
    c = np.empty((17, 23), np.float32)
    r.ref_matmul_view_f32(fp(row), 40, 0, 0, 1, fp(b), b.size, 0, 23, 1, 17, 40, 23, fp(c))
    v["expand_row"], v["expand_b"], v["expand_c"] = row, b, c

    # 4. contiguous 64x96x80 (the reference matmul_cpu path)
    a = oracle.uniform((64, 96), 48)
    b = oracle.uniform((96, 80), 49)
    c = np.empty((64, 80), np.float32)
    r.ref_matmul_f32(fp(a), fp(b), fp(c), 64, 96, 80)
    v["dense_a"], v["dense_b"], v["dense_c"] = a, b, c

    # 5. conv2d: [2,3,9,9] * [5,3,3,3], stride 2, pad 1, with bias
    x = oracle.normal((2, 3, 9, 9), 50)
    w = oracle.normal((5, 3, 3, 3), 51, std=(2 / 27) ** 0.5)
    bias = oracle.normal((5,), 52, std=0.1)
    out = np.empty((2, 5, 5, 5), np.float32)
    r.ref_conv2d_f32(fp(x), fp(w), fp(bias), fp(out), 2, 3, 9, 9, 5, 3, 3, 2, 1)
    v["conv_x"], v["conv_w"], v["conv_b"], v["conv_out"] = x, w, bias, out

    # 6. Linear (reference layout W_ref [in,out], bias [1,out]) forward + backward
    B, fin, fout = 12, 20, 7
    x = oracle.normal((B, fin), 53)
    w_ref = oracle.normal((fin, fout), 54, std=(2 / fin) ** 0.5)
    bias = oracle.normal((fout,), 55, std=0.1)
    dy = oracle.normal((B, fout), 56, std=0.01)
    y = np.empty((B, fout), np.float32)
    dx = np.empty((B, fin), np.float32)
    dw = np.empty((fin, fout), np.float32)
    db = np.empty((fout,), np.float32)
    r.ref_linear_f32(fp(x), fp(w_ref), fp(bias), fp(dy), B, fin, fout, fp(y), fp(dx), fp(dw), fp(db))
    v.update(lin_x=x, lin_w_ref=w_ref, lin_b=bias, lin_dy=dy, lin_y=y, lin_dx=dx, lin_dw_ref=dw,
             lin_db=db)

    # 7. conv2d backward through the reference's autograd (Conv2DBackward ->
    #    conv2d_backward_{input,weight,bias}_cpu): three images, so the
    #    per-image accumulation order of dW and db shows; stride 1 and 2.
    for tag, (n, c, h, wd, co, k, st, pad) in (("s1", (3, 4, 7, 6, 5, 3, 1, 1)),
                                                 ("s2", (3, 2, 9, 8, 3, 3, 2, 1))):
        x = oracle.normal((n, c, h, wd), 57 + st)
        w = oracle.normal((co, c, k, k), 59 + st, std=(2 / (c * k * k)) ** 0.5)
        ho, wo = oracle.conv_out(h, pad, k, st), oracle.conv_out(wd, pad, k, st)
        dy = oracle.normal((n, co, ho, wo), 61 + st, std=0.1)
        dx = np.empty_like(x)
        dw = np.empty_like(w)
        db = np.empty((co,), np.float32)
        r.ref_conv2d_bwd_f32(fp(x), fp(w), fp(dy), fp(dx), fp(dw), fp(db), n, c, h, wd, co, k, k,
                             st, pad)
        v.update({f"cbwd_{tag}_x": x, f"cbwd_{tag}_w": w, f"cbwd_{tag}_dy": dy,
                  f"cbwd_{tag}_dx": dx, f"cbwd_{tag}_dw": dw, f"cbwd_{tag}_db": db,
                  f"cbwd_{tag}_geom": np.array([st, pad], np.float32)})

    np.savez(OUT, **v)
    write_bin(v, OUT.with_suffix(".bin"))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
