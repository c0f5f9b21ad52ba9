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
