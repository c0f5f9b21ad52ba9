"""The C-ABI library on the CPU: it loads, exports every symbol include/qne.h declares, and
validates index.json before any device work (Index::validate, kernels/src/model.rs:51-86), with
the reference's error messages. No compute call is made here."""
import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

import qne as Q
import weights as W

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "qne.h").read_text()
    return sorted(set(re.findall(r"\b(qne_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = Q.load_library()
    names = declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n


def load_rc(index, weights, options=None):
    lib = Q.load_library()
    h = ctypes.c_void_p()
    ij = index.encode()
    w = np.ascontiguousarray(weights)
    rc = lib.qne_model_load(ij, len(ij), w.ctypes.data_as(ctypes.c_void_p), w.size,
                            json.dumps(options).encode() if options else None, 1, ctypes.byref(h))
    return rc, lib.qne_last_error().decode(), h


@pytest.fixture(scope="module")
def tiny():
    return W.synth_model("tiny", seed=1)


def mutate(index, f):
    ix = json.loads(index)
    f(ix)
    return json.dumps(ix)


def test_malformed_json_is_a_format_error(tiny):
    rc, msg, _ = load_rc("{not json", tiny[1])
    assert rc == Q.EFORMAT and "index.json" in msg


def test_tensor_outside_the_file(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["tensors"]["final_norm"].update(offset=len(buf)))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and msg == "invalid tensor range: final_norm"


def test_misaligned_tensor(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["tensors"]["layer0.post_norm"].update(offset=ix["tensors"]["layer0.post_norm"]["offset"] + 2))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and msg == "invalid tensor range: layer0.post_norm"


def test_wrong_tensor_size(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["tensors"]["layer1.conv_w"].update(bytes=ix["tensors"]["layer1.conv_w"]["bytes"] - 4))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and msg == "invalid tensor size: layer1.conv_w"


def test_wrong_matrix_shape(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["matrices"]["layer2.down"].update(rows=7))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and msg == "invalid matrix shape: layer2.down"


def test_missing_tensor(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["tensors"].pop("layer3.attn_norms"))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and msg == "invalid tensor size: layer3.attn_norms"


def test_format1_rejects_other_architectures(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix.update(format_version=1))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT
    assert msg == "unsupported model architecture: these kernels require Qwen3.5-0.8B or Qwen3.5-2B"


def test_unsupported_shapes_are_rejected(tiny):
    index, buf = tiny
    bad = mutate(index, lambda ix: ix["config"].update(head_dim=128))
    rc, msg, _ = load_rc(bad, buf)
    assert rc == Q.EFORMAT and "head_dim" in msg


def test_bad_options_are_rejected_before_device_work(tiny):
    rc, msg, _ = load_rc(tiny[0], tiny[1], {"max_context": 3})
    assert rc == Q.EINVAL and "max_context" in msg


def test_null_handle_calls_fail_cleanly():
    lib = Q.load_library()
    assert lib.qne_reset(None) == Q.EINVAL
    assert "null model handle" in lib.qne_last_error().decode()
    assert lib.qne_restore(None) == Q.EINVAL
    assert lib.qne_model_free(None) == Q.OK


def test_valid_model_reaches_device_initialisation(tiny):
    """Validation passes; what happens next depends on whether this host has a GPU."""
    rc, msg, h = load_rc(tiny[0], tiny[1])
    if rc == Q.OK:
        Q.load_library().qne_model_free(h)
    else:
        assert rc == Q.EDEVICE, msg


# ---- ModelTiles::validate (kernels/src/model.rs:101-109), checked at load after the index ----

GOLDEN = ROOT / "tests" / "golden"


def reference_profile(name):
    """The reference's own tile-profile files (kernels/profiles/*.json), kept as test data."""
    return json.loads((GOLDEN / name).read_text())


def tile(f16, tpr, rpw, rpt, splits):
    return dict(f16=f16, tpr=tpr, rpw=rpw, rpt=rpt, splits=splits)


def fast_tiles():
    """ModelTiles::fast() (model.rs:137-141)."""
    f32 = tile(False, 16, 4, 1, 1)
    return dict(gdn_in=tile(True, 16, 4, 4, 1), attn_in=tile(True, 4, 32, 4, 1), out=f32,
                gate_up=tile(True, 4, 16, 4, 1), down=f32, lm_head=tile(True, 4, 32, 4, 1))


def f32_tiles():
    """ModelTiles::f32() (model.rs:111-114)."""
    t = tile(False, 16, 4, 1, 1)
    return {k: dict(t) for k in ("gdn_in", "attn_in", "out", "gate_up", "down", "lm_head")}


def passes_tile_check(rc, msg):
    # a profile the reference accepts gets past validation; on a machine without a GPU the load
    # then stops at the device (and with one it loads)
    return rc in (Q.OK, Q.EDEVICE) and "tile" not in msg


@pytest.mark.parametrize("as_key", [True, False])
def test_reference_tile_profiles_validate(tiny, as_key):
    """model.rs:457-461: fast(), f32() and the shipped 2B profile are valid."""
    index, buf = tiny
    for profile in (fast_tiles(), f32_tiles(), reference_profile("tiles_uhd630_2b.json"),
                    reference_profile("tiles_uhd630_0.8b.json")):
        rc, msg, h = load_rc(index, buf, {"tiles": profile} if as_key else profile)
        assert passes_tile_check(rc, msg), msg
        if rc == Q.OK:
            Q.load_library().qne_model_free(h)


@pytest.mark.parametrize("kind,field,value", [("down", "splits", 0), ("lm_head", "tpr", 0)])
def test_invalid_tile_profiles_are_rejected(tiny, kind, field, value):
    """model.rs:462-465: the 2B profile with down.splits = 0, or with lm_head.tpr = 0, is invalid."""
    index, buf = tiny
    bad = reference_profile("tiles_uhd630_2b.json")
    bad[kind][field] = value
    rc, msg, _ = load_rc(index, buf, {"tiles": bad})
    assert rc == Q.EINVAL and msg.startswith("invalid kernel tile profile: Tile {"), msg
    t = bad[kind]
    assert msg == ("invalid kernel tile profile: Tile { f16: %s, tpr: %d, rpw: %d, rpt: %d, splits: %d }"
                   % ("true" if t["f16"] else "false", t["tpr"], t["rpw"], t["rpt"], t["splits"]))


@pytest.mark.parametrize("t,ok", [
    (tile(True, 64, 4, 8, 8), True),     # tpr * rpw = 256 is the largest allowed
    (tile(True, 64, 8, 1, 1), False),    # 512 threads per row group
    (tile(True, 3, 4, 1, 1), False),     # tpr not a power of two
    (tile(True, 4, 64, 1, 1), False),    # rpw above 32
    (tile(True, 4, 1, 1, 1), False),     # rpw below 2
    (tile(True, 4, 4, 16, 1), False),    # rpt above 8
    (tile(True, 4, 4, 1, 16), False),    # splits above 8
    (tile(False, 4, 4, 2, 1), False),    # f32 tiles take rpt = 1 ...
    (tile(False, 4, 4, 1, 2), False),    # ... and splits = 1
    (tile(False, 1, 2, 1, 1), True),
])
def test_tile_rules(tiny, t, ok):
    index, buf = tiny
    prof = f32_tiles()
    prof["gate_up"] = t
    rc, msg, h = load_rc(index, buf, {"tiles": prof})
    if ok:
        assert passes_tile_check(rc, msg), msg
        if rc == Q.OK:
            Q.load_library().qne_model_free(h)
    else:
        assert rc == Q.EINVAL and "invalid kernel tile profile" in msg, msg


def test_tile_profile_with_a_missing_field_is_rejected(tiny):
    index, buf = tiny
    prof = f32_tiles()
    del prof["down"]
    rc, msg, _ = load_rc(index, buf, {"tiles": prof})
    assert rc == Q.EINVAL and "down" in msg
    prof = f32_tiles()
    del prof["out"]["rpw"]
    rc, msg, _ = load_rc(index, buf, {"tiles": prof})
    assert rc == Q.EINVAL and "rpw" in msg


def test_index_errors_come_before_tile_errors(tiny):
    """model.rs:172-174: index.validate runs before tiles.validate."""
    index, buf = tiny
    bad_index = mutate(index, lambda ix: ix["tensors"]["final_norm"].update(offset=len(buf)))
    prof = f32_tiles()
    prof["down"]["splits"] = 0
    rc, msg, _ = load_rc(bad_index, buf, {"tiles": prof})
    assert rc == Q.EFORMAT and "tile" not in msg


def test_pack_sz_interleaves_scale_and_zero():
    """qne_pack_sz_q4g: the device layout of a q4 matrix's group parameters is (scale, zero) pairs."""
    lib = Q.load_library()
    rng = np.random.default_rng(3)
    scales = rng.integers(0, 2**16, size=37, dtype=np.uint16)
    zeros = rng.integers(0, 2**16, size=37, dtype=np.uint16)
    out = np.zeros(74, np.uint16)
    assert lib.qne_pack_sz_q4g(scales.ctypes.data, zeros.ctypes.data, 37, out.ctypes.data) == 0
    np.testing.assert_array_equal(out[0::2], scales)
    np.testing.assert_array_equal(out[1::2], zeros)
    assert lib.qne_pack_sz_q4g(None, zeros.ctypes.data, 37, out.ctypes.data) == Q.EINVAL
