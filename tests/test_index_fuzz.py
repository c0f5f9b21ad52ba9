"""Seeded mutation fuzz of index.json and of the load options (CPU): whatever the bytes, the loader
answers with an error code and a message (or, for a mutation that leaves a valid file, gets past
validation), never a crash. The reference parses the same file with serde and validates it in
Index::validate (kernels/src/model.rs:51-86). tests/test_sanitized_host.py runs this file again
against the AddressSanitizer + UndefinedBehaviorSanitizer build of the host code."""
import ctypes
import json
import random

import numpy as np
import pytest

import qne as Q
import weights as W

VALID = (Q.OK, Q.EINVAL, Q.ECONTEXT, Q.EDEVICE, Q.EFORMAT)


@pytest.fixture(scope="module")
def tiny():
    return W.synth_model("tiny", seed=1)


def load(index_bytes: bytes, buf, options: bytes | None = None):
    lib = Q.load_library()
    h = ctypes.c_void_p()
    w = np.ascontiguousarray(buf)
    rc = lib.qne_model_load(index_bytes, len(index_bytes), w.ctypes.data_as(ctypes.c_void_p), w.size, options, 1,
                            ctypes.byref(h))
    msg = lib.qne_last_error().decode("utf-8", "replace")
    if rc == Q.OK:
        lib.qne_model_free(h)
    return rc, msg


ODD_VALUES = [None, True, False, -1, 0, 1, 2 ** 31, 2 ** 32, 2 ** 53, 2 ** 64, -2 ** 63, 1.5, -0.0, 1e308, "", "x",
              "\u0000", [], {}, [1, 2], {"a": 1}]


def mutate_tree(obj, rng):
    """One structural change somewhere in the parsed JSON: a value replaced by an odd one, a key
    dropped or renamed, or a container emptied."""
    path = []
    node = obj
    while isinstance(node, (dict, list)) and node and rng.random() < 0.8:
        key = rng.choice(list(node.keys())) if isinstance(node, dict) else rng.randrange(len(node))
        path.append((node, key))
        node = node[key]
    if not path:
        return obj
    parent, key = path[-1]
    r = rng.random()
    if r < 0.6:
        parent[key] = rng.choice(ODD_VALUES)
    elif r < 0.8 and isinstance(parent, dict):
        del parent[key]
    elif isinstance(parent, dict):
        parent[key + "_"] = parent.pop(key)
    else:
        parent.clear()
    return obj


def mutate_bytes(data: bytes, rng) -> bytes:
    b = bytearray(data)
    for _ in range(rng.randint(1, 8)):
        op = rng.random()
        i = rng.randrange(len(b)) if b else 0
        if op < 0.4 and b:
            b[i] = rng.randrange(256)
        elif op < 0.6 and b:
            del b[i:i + rng.randint(1, 16)]
        elif op < 0.8:
            b[i:i] = bytes(rng.choice([b"{", b"}", b"[", b"]", b'"', b"\\", b"\\u", b"\\ud800", b",", b":", b"-",
                                       b"1e999", b"\xff", b"\x00", b"nul", b"tru"]))
        else:
            b = b[:i]
    return bytes(b)


@pytest.mark.parametrize("seed", range(6))
def test_structural_mutations_of_index_json(tiny, seed):
    index, buf = tiny
    rng = random.Random(1000 + seed)
    for _ in range(60):
        ix = mutate_tree(json.loads(index), rng)
        rc, msg = load(json.dumps(ix).encode(), buf)
        assert rc in VALID
        assert rc in (Q.OK, Q.EDEVICE) or msg


@pytest.mark.parametrize("seed", range(6))
def test_byte_mutations_of_index_json(tiny, seed):
    index, buf = tiny
    rng = random.Random(2000 + seed)
    for _ in range(80):
        rc, msg = load(mutate_bytes(index.encode(), rng), buf)
        assert rc in VALID
        assert rc in (Q.OK, Q.EDEVICE) or msg


def test_short_weights_and_deep_nesting(tiny):
    index, buf = tiny
    for cut in (0, 1, 255, len(buf) // 2, len(buf) - 1):
        rc, msg = load(index.encode(), buf[:cut])
        assert rc == Q.EFORMAT, (cut, msg)
    deep = b"[" * 100000 + b"]" * 100000
    rc, msg = load(deep, buf)
    assert rc in (Q.EFORMAT, Q.EINVAL) and msg
    rc, msg = load(b'{"format_version": 2, "tensors": ' + b'{"a": ' * 50000 + b'1' + b'}' * 50001, buf)
    assert rc in (Q.EFORMAT, Q.EINVAL) and msg


@pytest.mark.parametrize("seed", range(3))
def test_mutated_options_and_tile_profiles(tiny, seed):
    index, buf = tiny
    rng = random.Random(3000 + seed)
    base = {"max_context": 256, "tiles": {k: dict(f16=True, tpr=4, rpw=32, rpt=4, splits=1)
                                          for k in ("gdn_in", "attn_in", "out", "gate_up", "down", "lm_head")}}
    for _ in range(40):
        opts = mutate_tree(json.loads(json.dumps(base)), rng)
        rc, msg = load(index.encode(), buf, json.dumps(opts).encode())
        assert rc in VALID
        raw = mutate_bytes(json.dumps(base).encode(), rng)
        rc, msg = load(index.encode(), buf, raw.replace(b"\x00", b" "))
        assert rc in VALID
