"""Writes the golden fixtures of tests/golden/ from the reference's own host code.

The reference's host library (BlockManager, Workspace, dispatcher, validation, status mapping,
slot / budget helpers) is compiled from its sources in its CPU (STUB) mode into
oracle/_ref/libsca_ref.so by oracle/build_oracle.py, and driven through oracle/ref/ref_driver.cpp.
This script records seeded traces of that library as JSON. It runs only where /root/reference
exists; the fixtures it writes are plain data (inputs and the reference's outputs) and are what
the CPU test suite compares this repository's host layer and oracle against.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle.oracle as orc  # noqa: E402
from oracle import build_oracle  # noqa: E402


def _msg():
    return ctypes.create_string_buffer(2048)


# ---- BlockManager traces ------------------------------------------------------------------------

def bm_trace(seed: int, num_blocks: int, max_seqs: int, max_blocks: int, steps: int) -> dict:
    rng = np.random.default_rng(seed)
    bm = orc.RefBlockManager(num_blocks, max_seqs, max_blocks)
    held: list[int] = []
    ops, results = [], []
    for _ in range(steps):
        kind = rng.choice(["alloc", "alloc", "free", "append", "append", "reset", "sync"])
        if kind == "alloc":
            count = int(rng.integers(-1, 7))
            op = {"op": "allocate", "count": count}
            rc, ids, msg = bm.allocate(count)
            held.extend(ids)
            res = {"rc": rc, "ids": ids, "msg": msg}
        elif kind == "free":
            pool = list(held)
            pick = [int(x) for x in rng.choice(pool, size=min(len(pool), int(rng.integers(0, 4))),
                                                replace=False)] if pool else []
            extra = [int(x) for x in rng.integers(-2, num_blocks + 2, size=int(rng.integers(0, 2)))]
            ids = pick + extra
            if pick and rng.random() < 0.3:
                ids.append(pick[0])  # double free inside one call
            for i in pick:
                if i in held:
                    held.remove(i)
            op = {"op": "free", "ids": ids}
            bm.free(ids)
            res = {}
        elif kind == "append":
            seq = int(rng.integers(-1, max_seqs + 1))
            n = int(rng.integers(0, 4))
            ids = [int(x) for x in rng.integers(0, num_blocks, size=n)]
            op = {"op": "append_to_table", "seq": seq, "ids": ids}
            rc, msg = bm.append_to_table(seq, ids if n else None)
            res = {"rc": rc, "msg": msg}
        elif kind == "reset":
            seq = int(rng.integers(-1, max_seqs + 1))
            op = {"op": "reset_seq", "seq": seq}
            rc, msg = bm.reset_seq(seq)
            res = {"rc": rc, "msg": msg}
        else:
            op = {"op": "sync"}
            bm.sync()
            res = {}
        res["state"] = bm.state()
        ops.append(op)
        results.append(res)
    return {"create": [num_blocks, max_seqs, max_blocks], "ops": ops, "results": results}


# ---- dispatcher / validation ----------------------------------------------------------------------

CFG_FIELDS = ("backend", "layout", "causal", "return_lse", "scale", "softcap", "sliding_window",
              "num_splits", "allow_fallback", "has_cu_seqlens_q", "has_cu_seqlens_kv")


def ref_cfg(d: dict) -> orc.RefCfg:
    c = orc.RefCfg()
    for f in CFG_FIELDS:
        setattr(c, f, d.get(f, 0))
    return c


def ref_shape(s) -> orc.RefShape:
    return orc.RefShape(*s)


def dispatch_cases() -> list[dict]:
    R = orc.ref_lib()
    shapes = [
        (1, 1, 2048, 32, 8, 128), (16, 1, 4096, 32, 8, 128), (1, 1, 200, 8, 8, 64),
        (1, 1, 256, 8, 8, 64), (1, 16, 4096, 32, 8, 128), (1, 2, 16, 8, 8, 64),
        (1, 1024, 1024, 8, 8, 64), (1, 64, 64, 8, 8, 64), (1, 128, 128, 8, 8, 128),
        (1, 129, 129, 8, 8, 128), (1, 4096, 4096, 8, 8, 128), (4, 8192, 8192, 32, 8, 128),
        (1, 7, 7, 32, 8, 128), (1, 63, 63, 32, 8, 128), (1, 1000, 1000, 32, 8, 128),
        (2, 96, 160, 4, 2, 96), (1, 32, 512, 8, 1, 256), (1, 1, 1, 8, 8, 32),
        (1, 300, 300, 8, 2, 192), (1, 512, 4096, 16, 4, 160),
        # invalid shapes
        (1, 16, 16, 8, 8, 48), (0, 16, 16, 8, 8, 64), (1, 16, 16, 6, 4, 64),
        (1, 32, 16, 8, 8, 64), (1, 16, 16, 4, 8, 64),
    ]
    cfgs = [
        {}, {"causal": 1}, {"backend": 3}, {"backend": 4}, {"backend": 5}, {"backend": 1},
        {"backend": 2}, {"allow_fallback": 1}, {"backend": 4, "allow_fallback": 1},
        {"num_splits": 4}, {"layout": 1}, {"softcap": 30.0}, {"sliding_window": 128},
    ]
    out = []
    for s in shapes:
        for c in cfgs:
            backend, tile, ws = ctypes.c_int32(), (ctypes.c_int32 * 4)(), ctypes.c_uint64()
            buf = _msg()
            R.ref_select(ctypes.byref(ref_cfg(c)), ctypes.byref(ref_shape(s)), ctypes.byref(backend),
                         tile, ctypes.byref(ws), buf, 2048)
            ex = _msg()
            R.ref_explain(ctypes.byref(ref_cfg(c)), ctypes.byref(ref_shape(s)), ex, 2048)
            out.append({"cfg": c, "shape": list(s), "backend": backend.value, "tile": list(tile),
                        "workspace": ws.value, "reason": buf.value.decode(),
                        "explain": ex.value.decode()})
    return out


def validate_cases() -> list[dict]:
    R = orc.ref_lib()
    base = (2, 64, 64, 8, 8, 64)
    cases = [({}, base), ({"layout": 7}, base), ({}, (0, 64, 64, 8, 8, 64)),
             ({}, (2, 0, 64, 8, 8, 64)), ({}, (2, 64, 0, 8, 8, 64)), ({}, (2, 64, 64, 0, 8, 64)),
             ({}, (2, 64, 64, 8, 0, 64)), ({}, (2, 64, 64, 8, 8, 48)), ({}, (2, 64, 64, 8, 8, 512)),
             ({}, (2, 64, 64, 12, 8, 64)), ({"causal": 1}, (2, 65, 64, 8, 8, 64)),
             ({}, (2, 64, 64, 4, 8, 64)), ({"sliding_window": 16}, base),
             ({"softcap": -1.0}, base), ({"softcap": 20.0, "backend": 4}, base),
             ({"softcap": 20.0, "backend": 3}, base), ({"softcap": 20.0}, base),
             ({"scale": -0.5}, base), ({"num_splits": -2}, base),
             ({"has_cu_seqlens_q": 1}, base), ({"has_cu_seqlens_q": 1, "has_cu_seqlens_kv": 1}, base),
             ({"causal": 1}, (1, 1, 1, 1, 1, 32)), ({}, (1, 1, 1, 32, 8, 256)),
             ({"softcap": 5.0, "backend": 1}, base), ({"softcap": 5.0, "backend": 2}, base),
             ({"softcap": 5.0, "backend": 5}, base)]
    out = []
    for c, s in cases:
        buf = _msg()
        code = R.ref_validate(ctypes.byref(ref_cfg(c)), ctypes.byref(ref_shape(s)), buf, 2048)
        scale = R.ref_effective_scale(ctypes.byref(ref_cfg(c)), ctypes.byref(ref_shape(s)))
        out.append({"cfg": c, "shape": list(s), "code": code, "message": buf.value.decode(),
                    "effective_scale": scale})
    for d in (32, 64, 96, 128, 160, 192, 256):
        for sc in (0.0, 0.125, 0.3):
            c = {"scale": sc}
            s = (1, 1, 1, 1, 1, d)
            out.append({"cfg": c, "shape": list(s), "code": 0, "message": "ok",
                        "effective_scale": R.ref_effective_scale(ctypes.byref(ref_cfg(c)),
                                                                 ctypes.byref(ref_shape(s)))})
    return out


def varlen_cases() -> list[dict]:
    R = orc.ref_lib()
    cases = [([0, 3, 10, 11], 3), ([0, 5], 1), ([1, 5], 1), ([0, 5, 5], 2), ([0, 5, 4], 2),
             ([0, 1, 8, 71, 1071], 4), ([0], 0), ([0, 2], -1)]
    out = []
    for cu, batch in cases:
        arr = np.asarray(cu, dtype=np.int32)
        mx = ctypes.c_int64(-1)
        buf = _msg()
        code = R.ref_validate_varlen(arr.ctypes.data, batch, ctypes.byref(mx), buf, 2048)
        out.append({"cu": cu, "batch": batch, "code": code, "max_seq": mx.value if code == 0 else None,
                    "message": buf.value.decode()})
    null = _msg()
    code = R.ref_validate_varlen(None, 2, None, null, 2048)
    out.append({"cu": None, "batch": 2, "code": code, "max_seq": None,
                "message": null.value.decode()})
    return out


def status_cases() -> dict:
    R = orc.ref_lib()
    codes = [0] + list(range(2001, 2011)) + [1999, 3000]
    names = {c: R.ref_status_name(c).decode() for c in codes}
    sci = {c: R.ref_to_sci_code(c) for c in codes}
    made = []
    for c, detail in [(2007, "out of blocks"), (2001, "head_dim=48"), (2009, ""), (0, "fine")]:
        buf = _msg()
        st = R.ref_make_status(c, detail.encode(), buf, 2048)
        made.append({"code": c, "detail": detail, "sci_code": st, "message": buf.value.decode()})
    extract = {m: R.ref_extract_code(m.encode()) for m in
               ["[SCA-2007] x", "no code", "prefix [SCA-2005] mid", "[SCA-] bad", "[SCA-2010]"]}
    backends = {k: R.ref_backend_name(k).decode() for k in range(-1, 8)}
    layouts = {k: R.ref_layout_name(k).decode() for k in range(-1, 3)}
    parse = {}
    for name in ["auto", "naive", "tiled", "flash", "decode", "paged", "Flash", "", "fa2"]:
        out = ctypes.c_int32(-1)
        ok = R.ref_parse_backend(name.encode(), ctypes.byref(out))
        parse[name] = out.value if ok else None
    hdi = {d: R.ref_supported_head_dim_index(d) for d in
           [0, 16, 32, 48, 64, 96, 128, 160, 192, 256, 257, 512]}
    smem = []
    for args in [(128, 2, 64, 64, 4, 2), (64, 2, 64, 64, 4, 2), (256, 2, 32, 32, 4, 2),
                 (160, 2, 64, 32, 8, 2), (128, 4, 64, 64, 4, 3), (0, 2, 64, 64, 4, 2),
                 (128, 2, 0, 64, 4, 2)]:
        smem.append({"args": list(args), "bytes": R.ref_tile_smem_bytes_flash(*args)})
    return {"names": names, "sci_codes": sci, "make_status": made, "extract": extract,
            "backend_names": backends, "layout_names": layouts, "parse_backend": parse,
            "head_dim_index": hdi, "tile_smem_bytes_flash": smem}


def kv_helper_cases() -> dict:
    R = orc.ref_lib()
    slots = []
    for row, start, n, bs, mb in [([3, 1, 0, -1], 17, 5, 8, 4), ([3, 1, 0, -1], 48, 1, 16, 4),
                                  ([3, 1, 0, -1], 0, 24, 8, 4), ([3, 1, 0, -1], 30, 5, 8, 4),
                                  ([5, 9], 0, 1, 1, 2), ([7, 2, 4], 10, 30, 16, 3),
                                  ([7, 2, 4], 10, 40, 16, 3), ([0], 0, 0, 16, 1),
                                  ([0], 0, 4, 0, 1), ([12, 40, 3, 8], 63, 2, 32, 4)]:
        arr = np.asarray(row, dtype=np.int32)
        out = np.zeros(max(n, 1), dtype=np.int32)
        buf = _msg()
        code = R.ref_compute_slot_mapping(arr.ctypes.data, start, n, bs, mb, out.ctypes.data,
                                          buf, 2048)
        slots.append({"row": row, "start": start, "n": n, "bs": bs, "max_blocks": mb,
                      "code": code, "slots": out[:n].tolist() if code == 0 else None,
                      "message": buf.value.decode() if code else ""})
    kv_bytes = []
    for cfg in [(32, 8, 128, 16, 2048, 64, 1), (36, 8, 128, 16, 34500, 64, 2),
                (1, 8, 128, 16, 34500, 64, 2), (2, 4, 64, 8, 100, 4, 0),
                (0, 8, 128, 16, 10, 1, 1), (1, 0, 128, 16, 10, 1, 1), (1, 8, 48, 16, 10, 1, 1),
                (1, 8, 128, 12, 10, 1, 1), (1, 8, 128, 16, 0, 1, 1), (1, 8, 128, 16, 10, 0, 1),
                (1, 8, 128, 16, 10, 1, 4), (1, 8, 128, 1, 7, 1, 1), (1, 8, 128, 64, 7, 1, 2)]:
        buf = _msg()
        v = R.ref_kv_cache_bytes(*cfg, buf, 2048)
        kv_bytes.append({"cfg": list(cfg), "value": v, "message": buf.value.decode() if v < 0 else ""})
    budget = []
    for args in [(32, 8, 128, 16, 1, 3221225472), (32, 8, 128, 16, 1, 1 << 30),
                 (32, 8, 128, 16, 0, 3221225472), (1, 8, 128, 16, 2, 100),
                 (0, 8, 128, 16, 1, 1 << 20), (36, 8, 128, 16, 2, 200 << 30)]:
        budget.append({"args": list(args), "value": R.ref_max_blocks_for_budget(*args)})
    splits = [{"seq_kv": s, "sms": m, "value": R.ref_splits_for(s, m)}
              for s in (0, 1, 511, 512, 513, 2048, 4096, 8192, 1 << 20)
              for m in (0, 1, 4, 36, 256)]
    partial = [{"args": list(a), "value": R.ref_partial_elements(*a)}
               for a in [(16, 32, 8, 128), (1, 1, 1, 32), (64, 32, 16, 128)]]
    return {"slot_mapping": slots, "kv_cache_bytes": kv_bytes, "max_blocks_for_budget": budget,
            "splits_for": splits, "partial_elements": partial}


def workspace_trace() -> list[dict]:
    R = orc.ref_lib()
    traces = []
    for size, ops in [
        (4096, [("slice", 0, 256, 256), ("slice", 256, 512, 256), ("slice", 0, 256, 256),
                ("slice", 128, 64, 256), ("slice", 100, 64, 256), ("slice", 128, 64, 64),
                ("slice", 3840, 512, 256), ("slice", 4096, 1, 256), ("slice", 512, 0, 256),
                ("slice", 768, 256, 0), ("reset",), ("slice", 128, 64, 64), ("slice", 0, 4096, 256)]),
        (1000, [("slice", 0, 1000, 8), ("slice", 0, 1001, 8), ("slice", 992, 8, 8)]),
    ]:
        buf = _msg()
        h = R.ref_ws_create(size, buf, 2048)
        results = []
        for op in ops:
            if op[0] == "reset":
                results.append({"op": "reset", "code": R.ref_ws_reset(h)})
            else:
                rel = ctypes.c_uint64(0)
                m = _msg()
                code = R.ref_ws_slice(h, op[1], op[2], op[3], ctypes.byref(rel), m, 2048)
                results.append({"op": "slice", "args": list(op[1:]), "code": code,
                                "offset": rel.value if code == 0 else None,
                                "message": m.value.decode() if code else ""})
            results[-1]["peak"] = R.ref_ws_peak(h)
            results[-1]["slices"] = R.ref_ws_slices(h)
        R.ref_ws_destroy(h)
        traces.append({"bytes": size, "results": results})
    m = _msg()
    h = R.ref_ws_create(0, m, 2048)
    traces.append({"bytes": 0, "create_failed": h is None, "message": m.value.decode()})
    return traces


def main() -> None:
    if not os.path.isdir("/root/reference"):
        raise SystemExit("the reference checkout is not present; fixtures are generated only here")
    build_oracle.build_oracle()
    build_oracle.build_reference()
    if orc.ref_lib() is None:
        raise SystemExit("oracle/_ref/libsca_ref.so did not build")
    fixtures = {
        "block_manager_traces.json": [bm_trace(s, nb, ms, mb, st) for s, nb, ms, mb, st in
                                      [(1, 16, 4, 8, 80), (2, 8, 2, 8, 60), (3, 32, 6, 12, 120),
                                       (4, 5, 3, 3, 60), (5, 48, 8, 16, 120)]],
        "dispatch.json": dispatch_cases(),
        "validate.json": validate_cases(),
        "varlen.json": varlen_cases(),
        "status.json": status_cases(),
        "kv_helpers.json": kv_helper_cases(),
        "workspace.json": workspace_trace(),
    }
    for name, data in fixtures.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, indent=None, separators=(",", ":"), sort_keys=True)
        print(name, os.path.getsize(os.path.join(HERE, name)), "bytes")


if __name__ == "__main__":
    main()
