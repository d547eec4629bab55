"""Per-path disable switches (fireprot_amd.switches), each in a fresh process.

The reference turns its HIP paths off from the environment and tests the
predicate's rejection in a child process (e.g.
tests/operators/test_ck_attention_exact1536.py:52-62): the flags are read at
import, so each case runs ``python -c`` with the flag set.  In the child a
signature that passes every other check of the candidate is built, and the
predicate must reject it with the flag's reason; the dispatch then runs the
caller's native function.
"""
from __future__ import annotations

import json
import os
import pathlib
import subprocess
import sys

import pytest

from fireprot_amd import switches

ROOT = pathlib.Path(__file__).resolve().parents[1]

CHILD = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
from fireprot_amd import (attention_gate, layer_norm, openfold3, qkv_projection, switches,
                          transition, triangle_attention as ta, triangle_multiplication as tm)
from fireprot_amd.registry import OperationSignature, registry

def sig(operation, dtype="float32", shape=(512, 4, 1536, 32), **attributes):
    return OperationSignature.create(
        operation=operation, device_type="cuda", architecture="gfx950", dtype=dtype,
        shape=shape, layout="strided", mode="inference", attributes=attributes)

def safe(fn):
    try:
        return fn()
    except Exception as error:  # the check after the flag needs real objects
        return ["error", type(error).__name__]

n = 1536
core = sig(ta.OPERATION, bias_count=1, bias_shapes=repr(((1, 4, n, n),)),
           qkv_strides=repr(((n * 128, 32, 128, 1),) * 3), ck_tile_compatible=True)
block = sig(ta.BLOCK_OPERATION, shape=(n, n, 128), eligible=True, reason="", ending=False)
result = {
    "core": ta._supports_core(core),
    "block": ta._supports_block(block),
    "block_bf16": ta._supports_block(sig(ta.BLOCK_OPERATION, dtype="bfloat16",
                                          shape=(n, n, 128), eligible=True),
                                      dtype="bfloat16"),
    "trimul": tm._supports(sig(tm.OPERATION, shape=(n, n, 128), c_z=128, c_hidden=128,
                               eligible=True)),
    "transition": transition._supports(sig(transition.OPERATION, shape=(n, n, 128),
                                           expansion=4, eligible=True)),
    "openfold3": openfold3.AttentionDispatcher(None)._eligible(None, None, None, None),
    "layer_norm": layer_norm.eligible(None, None),
    "qkv": safe(lambda: qkv_projection.supported(None, None, None, True)),
    "gate": safe(lambda: attention_gate.supported(None, None, None)),
    "state": switches.manifest(),
}
registry.clear_runtime_state()
if result["core"] is not True:  # a selected HIP candidate would need real tensors
    result["dispatch"] = registry.dispatch(core, lambda **_: "native")
print(json.dumps({k: (list(v) if isinstance(v, tuple) else v) for k, v in result.items()}))
"""


def _child(env_update: dict) -> dict:
    env = {k: v for k, v in os.environ.items() if not k.startswith("FPX_DISABLE")}
    env.update(env_update)
    out = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], env=env, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return json.loads(out.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("flag,key", [
    ("FPX_DISABLE_ATTENTION", "core"),
    ("FPX_DISABLE_BLOCK", "block"),
    ("FPX_DISABLE_BLOCK_BF16", "block_bf16"),
    ("FPX_DISABLE_TRIANGLE_MULTIPLICATION", "trimul"),
    ("FPX_DISABLE_TRANSITION", "transition"),
    ("FPX_DISABLE_OPENFOLD3_ATTENTION", "openfold3"),
    ("FPX_DISABLE_LAYER_NORM", "layer_norm"),
])
def test_each_flag_rejects_its_candidate_with_a_reason(flag, key):
    r = _child({flag: "1"})
    assert r[key] == [False, f"disabled by {flag}=1"]
    assert r["state"][flag] is True
    assert sum(r["state"].values()) == 1  # no other path is touched
    if key == "core":
        assert r["dispatch"] == "native"


@pytest.mark.parametrize("flag,key", [("FPX_DISABLE_QKV_PROJECTION", "qkv"),
                                      ("FPX_DISABLE_ATTENTION_GATE", "gate")])
def test_stage_hook_flags(flag, key):
    assert _child({flag: "1"})[key] is False


def test_without_flags_the_predicates_reach_their_own_checks():
    r = _child({})
    assert not any(r["state"].values())
    # no flag: the first rejection is a real check (the library may or may
    # not load on this host, but no reason names a flag)
    for key in ("core", "block", "block_bf16", "trimul", "transition"):
        assert r[key] is True or "disabled by" not in r[key][1], (key, r[key])
    assert r["openfold3"] == [False, "no HIP kernel"]


def test_disable_all_and_values_other_than_one():
    r = _child({"FPX_DISABLE_ALL": "1"})
    assert all(r["state"].values())
    assert r["core"] == [False, "disabled by FPX_DISABLE_ALL=1"]
    r = _child({"FPX_DISABLE_ATTENTION": "0", "FPX_DISABLE_BLOCK": "yes"})
    assert not any(r["state"].values())


def test_every_flag_is_listed():
    assert set(switches.FLAGS) == {
        "FPX_DISABLE_ATTENTION", "FPX_DISABLE_BLOCK", "FPX_DISABLE_BLOCK_BF16",
        "FPX_DISABLE_TRIANGLE_MULTIPLICATION", "FPX_DISABLE_TRANSITION",
        "FPX_DISABLE_OPENFOLD3_ATTENTION", "FPX_DISABLE_LAYER_NORM",
        "FPX_DISABLE_QKV_PROJECTION", "FPX_DISABLE_ATTENTION_GATE"}
