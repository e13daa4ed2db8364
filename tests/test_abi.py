"""The C ABI library loads and exports every entry point include/t5hip.h declares (CPU only).

Also exercises the host-side error paths that run before any device work, the way the
reference tests a missing-assets Embedder (src/tests.rs:480-491).
"""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from witchcraft_amd import _lib, synth
from witchcraft_amd.encoder import T5ModelBuilder, config_from_json

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "t5hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t5h_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_surface():
    fns = header_functions()
    for need in ("t5h_create", "t5h_destroy", "t5h_encode", "t5h_encode_normalized",
                 "t5h_last_error", "t5h_q4k_dequant_f32", "t5h_layer_forward", "t5h_ffn_block"):
        assert need in fns


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing
    # and the ctypes binding covers exactly the header
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_config_defaults_and_json():
    c = _lib.T5HConfig()
    _lib.check(_lib.lib.t5h_config_xtr_base(C.byref(c)))
    assert (c.vocab_size, c.d_model, c.d_kv, c.d_ff, c.num_layers, c.num_heads) == (32128, 768, 64, 2048, 12, 12)
    assert c.relative_attention_num_buckets == 32 and c.relative_attention_max_distance == 128
    j = config_from_json(synth.config_json())
    assert j.feed_forward_gated == 1 and j.vocab_size == 32128 and abs(j.layer_norm_epsilon - 1e-6) < 1e-12
    with pytest.raises(ValueError):
        config_from_json(b'{"d_model": 768}')


def _create(buf: bytes, cfg):
    h = C.c_void_p()
    arr = np.frombuffer(buf, np.uint8) if buf else np.zeros(1, np.uint8)
    rc = _lib.lib.t5h_create(np.ascontiguousarray(arr), len(buf), C.byref(cfg), 0, C.byref(h))
    return rc, h


def test_create_rejects_bad_inputs_before_device_work():
    c = _lib.T5HConfig()
    _lib.lib.t5h_config_xtr_base(C.byref(c))
    rc, h = _create(b"", c)
    assert rc == _lib.T5H_ERR_FORMAT and not h.value
    rc, _ = _create(b"NOTGGUF" * 10, c)
    assert rc == _lib.T5H_ERR_FORMAT
    assert b"magic" in _lib.lib.t5h_last_error()
    bad = _lib.T5HConfig()
    _lib.lib.t5h_config_xtr_base(C.byref(bad))
    bad.d_kv = 32
    rc, _ = _create(b"GGUF", bad)
    assert rc == _lib.T5H_ERR_INVALID
    # truncated tensor table
    img = synth.make_model(synth.small_config(), seed=0)
    small = config_from_json(synth.small_config())
    rc, _ = _create(img[:200], small)
    assert rc == _lib.T5H_ERR_FORMAT


def test_builder_without_assets(tmp_path):
    with pytest.raises(FileNotFoundError, match="CONFIG"):
        T5ModelBuilder.load(tmp_path)
    (tmp_path / "config.json").write_bytes(synth.config_json())
    b, tok = T5ModelBuilder.load(tmp_path)
    assert tok is None
    with pytest.raises(FileNotFoundError, match="MODEL"):
        b.build_encoder(0, tmp_path)


def test_null_handles_are_errors():
    assert _lib.lib.t5h_synchronize(None) == _lib.T5H_ERR_INVALID
    assert _lib.lib.t5h_stream(None) is None
    _lib.lib.t5h_destroy(None)
