"""The host layer (libsca_host.so through include/sca_capi.h) against the reference's own host
code: the golden fixtures of tests/golden/ were recorded from the reference compiled in its CPU
mode (tests/golden/make_golden.py). CPU only: nothing here launches a kernel."""

from __future__ import annotations

import json
import os
import struct

import pytest

from sca_amd import host as H

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def cfg_from(d: dict) -> H.AttentionConfig:
    import numpy as np

    cu = np.array([0, 1], dtype=np.int32)
    return H.AttentionConfig(
        backend=d.get("backend", 0), layout=d.get("layout", 0), causal=bool(d.get("causal", 0)),
        return_lse=bool(d.get("return_lse", 0)), scale=d.get("scale", 0.0),
        softcap=d.get("softcap", 0.0), sliding_window=d.get("sliding_window", 0),
        num_splits=d.get("num_splits", 0), allow_fallback=bool(d.get("allow_fallback", 0)),
        cu_seqlens_q=cu if d.get("has_cu_seqlens_q") else None,
        cu_seqlens_kv=cu if d.get("has_cu_seqlens_kv") else None)


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ---- BlockManager: bit-exact state after every operation ----------------------------------------

@pytest.mark.parametrize("index", range(5))
def test_block_manager_trace_matches_reference(index):
    trace = load("block_manager_traces.json")[index]
    nb, seqs, maxb = trace["create"]
    bm = H.BlockManager(nb, seqs, maxb, device=H.HOST)
    for step, (op, want) in enumerate(zip(trace["ops"], trace["results"])):
        tag = f"step {step} {op}"
        kind = op["op"]
        if kind == "allocate":
            try:
                ids = bm.allocate(op["count"]).tolist()
                rc, msg = 0, ""
            except H.ScaError as e:
                ids, rc, msg = [], e.code, e.message
            assert rc == want["rc"], tag
            assert ids == want["ids"], tag
            assert msg == want["msg"], tag
        elif kind == "free":
            bm.free(op["ids"])
        elif kind == "append_to_table":
            try:
                bm.append_to_table(op["seq"], op["ids"])
                rc, msg = 0, ""
            except H.ScaError as e:
                rc, msg = e.code, e.message
            assert rc == want["rc"], tag
            if rc:
                assert msg == want["msg"], tag
        elif kind == "reset_seq":
            try:
                bm.reset_seq(op["seq"])
                rc, msg = 0, ""
            except H.ScaError as e:
                rc, msg = e.code, e.message
            assert rc == want["rc"], tag
            if rc:
                assert msg == want["msg"], tag
        else:
            bm.sync()
        assert bm.state() == want["state"], tag


def test_block_manager_device_table_follows_sync_on_host_device():
    bm = H.BlockManager(8, 2, 4, device=H.HOST)
    ids = bm.allocate(3)
    bm.append_to_table(1, ids)
    assert bm.table_device().tolist() == [-1] * 8
    bm.sync()
    assert bm.table_device().tolist() == bm.table().tolist()


# ---- dispatcher ---------------------------------------------------------------------------------

def _rule(reason: str) -> str:
    """The decision part of a reason string (before the capability verdict and table tag)."""
    for cut in (" => unsupported(", " [table="):
        if cut in reason:
            reason = reason[: reason.index(cut)]
    return reason


def test_dispatch_matches_reference_rules():
    cases = load("dispatch.json")
    for case in cases:
        cfg = cfg_from(case["cfg"])
        got = H.select(cfg, H.AttentionShape(*case["shape"]))
        tag = f"{case['shape']} {case['cfg']}"
        if case["reason"].startswith("invalid: "):
            assert got["backend"] == 0, tag
            assert got["reason"] == case["reason"], tag
            continue
        want_rule = _rule(case["reason"])
        got_rule = _rule(got["reason"])
        if case["backend"] == 2 and case["cfg"].get("backend", 0) == 0:
            # The MI355X table serves the reference's "short sequence" rule on flash.
            assert got["backend"] == 3, tag
            assert "short sequence" in got_rule and want_rule.split(" => ")[0] == got_rule.split(" => ")[0], tag
            continue
        assert got["backend"] == case["backend"], tag
        assert got_rule == want_rule, tag
        # Without a GPU every backend refuses; the refusal names the backend and the table.
        assert f"=> unsupported({H.backend_name(got['backend'])})" in got["reason"], tag
        assert "[table=r0-mi355x" in got["reason"] or "no fallback backend" in got["reason"], tag


def test_explain_format_matches_reference():
    for case in load("dispatch.json")[:40]:
        text = H.explain(cfg_from(case["cfg"]), H.AttentionShape(*case["shape"]))
        want = case["explain"]
        for field in ("backend=", "; tile={bm=", ",bn=", ",warps=", ",stages=", ",tma=off}",
                      "; workspace=", " B; reason="):
            assert field in text and field in want, (field, text)


# ---- validation ---------------------------------------------------------------------------------

def test_validate_matches_reference():
    for case in load("validate.json"):
        cfg = cfg_from(case["cfg"])
        shape = H.AttentionShape(*case["shape"])
        code, detail = H.validate(cfg, shape)
        tag = f"{case['shape']} {case['cfg']}"
        assert code == case["code"], tag
        if code:
            assert f"[SCA-{code}] {detail}" == case["message"] or detail == case["message"], tag
        assert f32_bits(H.effective_scale(cfg, shape)) == f32_bits(case["effective_scale"]), tag


def test_validate_varlen_matches_reference():
    for case in load("varlen.json"):
        if case["cu"] is None:
            code, _, msg = H.validate_varlen([], case["batch"])
            code2 = H.host_lib().sca_validate_varlen(None, case["batch"], None)
            assert code2 == case["code"]
            assert H.host_lib().sca_last_error().decode() == case["message"]
            continue
        code, mx, msg = H.validate_varlen(case["cu"], case["batch"])
        assert code == case["code"], case
        if code == 0:
            assert mx == case["max_seq"], case
        else:
            assert msg == case["message"], case


# ---- status / names -----------------------------------------------------------------------------

def test_status_mapping_matches_reference():
    st = load("status.json")
    for code, name in st["names"].items():
        assert H.status_name(int(code)) == name
    for code, sci in st["sci_codes"].items():
        assert H.to_sci_code(int(code)) == sci
    for m in st["make_status"]:
        sci, msg = H.make_status(m["code"], m["detail"])
        assert (sci, msg) == (m["sci_code"], m["message"])
    for msg, code in st["extract"].items():
        assert H.extract_code(msg) == code
    for kind, name in st["backend_names"].items():
        assert H.backend_name(int(kind)) == name
    for lay, name in st["layout_names"].items():
        assert H.layout_name(int(lay)) == name
    for name, kind in st["parse_backend"].items():
        assert H.parse_backend(name) == kind
    for d, idx in st["head_dim_index"].items():
        assert H.supported_head_dim_index(int(d)) == idx
    for s in st["tile_smem_bytes_flash"]:
        assert H.host_lib().sca_tile_smem_bytes_flash(*s["args"]) == s["bytes"]


# ---- KV helpers ---------------------------------------------------------------------------------

def test_slot_mapping_matches_reference():
    for c in load("kv_helpers.json")["slot_mapping"]:
        try:
            got = H.compute_slot_mapping(c["row"], c["start"], c["n"], c["bs"], c["max_blocks"])
            code, msg = 0, ""
        except H.ScaError as e:
            got, code, msg = None, e.code, e.message
        assert code == c["code"], c
        if code == 0:
            assert got.tolist() == c["slots"], c
        else:
            assert msg == c["message"], c


def test_kv_bytes_and_budget_match_reference():
    kv = load("kv_helpers.json")
    for c in kv["kv_cache_bytes"]:
        layers, heads, d, bs, nb, seqs, dtype = c["cfg"]
        cfg = H.KVCacheConfig(layers, heads, d, bs, nb, seqs,
                              {0: "f32", 1: "f16", 2: "bf16", 4: "i32"}[dtype])
        try:
            got = H.kv_cache_bytes(cfg)
        except H.ScaError as e:
            assert c["value"] == -e.code and e.message == c["message"], c
            continue
        assert got == c["value"], c
    for c in kv["max_blocks_for_budget"]:
        layers, heads, d, bs, dtype, budget = c["args"]
        cfg = H.KVCacheConfig(layers, heads, d, bs, 0, 1, {0: "f32", 1: "f16", 2: "bf16"}[dtype])
        assert H.max_blocks_for_budget(cfg, budget) == c["value"], c


def test_reference_kv_known_answers():
    """test_kv_cache.cpp:38-81 of the reference."""
    cfg = H.KVCacheConfig(32, 8, 128, 16, 1536, 4, "f16")
    b = H.kv_cache_bytes(cfg)
    assert b == 3221225472 and b // 1536 == 2097152
    assert H.max_blocks_for_budget(cfg, b) == 1536
    assert H.max_blocks_for_budget(cfg, b // 2) == 768
    assert H.compute_slot_mapping([3, 1, 0, -1], 17, 5, 16, 4).tolist() == [17, 18, 19, 20, 21]
    H.compute_slot_mapping([3, 1, 0, -1], 22, 5, 16, 4)
    with pytest.raises(H.ScaError) as e:
        H.compute_slot_mapping([3, 1, 0, -1], 48, 1, 16, 4)
    assert "empty" in e.value.message


# ---- workspace ----------------------------------------------------------------------------------

def test_workspace_matches_reference():
    for trace in load("workspace.json"):
        if trace["bytes"] == 0:
            with pytest.raises(H.ScaError) as e:
                H.Workspace(0)
            assert e.value.message == trace["message"]
            continue
        ws = H.Workspace(trace["bytes"])
        for r in trace["results"]:
            if r["op"] == "reset":
                ws.reset()
            else:
                try:
                    off, code, msg = ws.slice(*r["args"]), 0, ""
                except H.ScaError as e:
                    off, code, msg = None, e.code, e.message
                assert code == r["code"], r
                if code == 0:
                    assert off == r["offset"], r
                else:
                    assert msg == r["message"], r
            assert ws.peak == r["peak"] and ws.slices == r["slices"], r
