"""Hybrid-dequant numerics on the GPU (t5h_set_numerics(T5H_NUMERICS_HYBRID)): the Q8_K
activation quantizer, the Q4_K x Q8_K integer dot products, and whole forwards against the
oracle's hybrid variant (src/fused_matmul.rs:27-59,138-177)."""
import numpy as np
import pytest

from oracle import oracle as orc
from witchcraft_amd import synth
from witchcraft_amd.quantize import quantize_q4k

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def enc():
    from witchcraft_amd import encoder
    return encoder


def _q8k_rows():
    rng = np.random.default_rng(61)
    rows = [rng.standard_normal(768), rng.standard_normal(768) * 1e-3, np.zeros(768),
            rng.uniform(0.1, 2.0, 768), -rng.uniform(0.1, 2.0, 768), rng.standard_normal(768) * 300]
    r = rng.standard_normal(768)
    r[[10, 40]] = [-5.0, 5.0]        # tie on |x|: the first (negative) one sets the scale
    r[300] = 5.0
    r[290] = 5.0                     # tie inside the second block, positive first
    r[600:] = 0.0                    # last block partly zero
    rows.append(r)
    r = np.round(rng.standard_normal(768) * 8) / 8  # many products exactly on rounding ties
    rows.append(r)
    return np.stack(rows).astype(np.float32)


def test_q8k_quantize_bit_exact(enc):
    x = _q8k_rows()
    got = enc.q8k_quantize(x)
    want = np.stack([orc.q8k_quantize(r) for r in x])
    assert np.array_equal(got, want)


def test_q4k_q8k_matmul_vs_oracle(enc):
    rng = np.random.default_rng(62)
    K, N, T = 768, 128, 20
    w = quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x8 = enc.q8k_quantize((rng.standard_normal((T, K))).astype(np.float32))
    got = enc.q4k_q8k_matmul(w, x8, K)
    want = np.array([[orc.q4k_q8k_vec_dot(K, w[n], x8[t]) for n in range(N)] for t in range(T)], np.float32)
    # integer parts are exact; only the f32 combination order of the block terms differs
    wd = orc.q4k_dequant(w).reshape(N, K).astype(np.float64)
    xd = np.stack([_q8k_dequant(r) for r in x8])
    scale = np.abs(xd) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-30)


def _q8k_dequant(row: np.ndarray) -> np.ndarray:
    b = row.reshape(-1, 292)
    d = b[:, :4].copy().view(np.float32)[:, 0]
    q = b[:, 4:260].view(np.int8).astype(np.float64)
    return (q * d[:, None]).reshape(-1)


def test_q4k_q8k_exact_when_the_float_terms_are_exact(enc):
    """d = 2^-8, dmin = 2^-10 in f16 and d8 = 1 make every block term an exact float, so the
    result is the exact integer expression whatever the summation order."""
    rng = np.random.default_rng(63)
    K, N, T = 512, 64, 5
    blocks = np.zeros((N, K // 256, 144), np.uint8)
    blocks[:, :, 0:2] = np.array([2.0 ** -8], np.float16).view(np.uint8)
    blocks[:, :, 2:4] = np.array([2.0 ** -10], np.float16).view(np.uint8)
    blocks[:, :, 4:16] = rng.integers(0, 256, (N, K // 256, 12))
    blocks[:, :, 16:] = rng.integers(0, 256, (N, K // 256, 128))
    w = blocks.reshape(N, -1)
    x8 = np.zeros((T, K // 256, 292), np.uint8)
    x8[:, :, 0:4] = np.array([1.0], np.float32).view(np.uint8)
    q = rng.integers(-128, 128, (T, K // 256, 256)).astype(np.int8)
    x8[:, :, 4:260] = q.view(np.uint8)
    x8[:, :, 260:] = q.reshape(T, K // 256, 16, 16).astype(np.int32).sum(-1).astype(np.int16).view(np.uint8).reshape(T, K // 256, 32)
    x8 = x8.reshape(T, -1)
    got = enc.q4k_q8k_matmul(w, x8, K)
    exact = q.reshape(T, K).astype(np.float64) @ orc.q4k_dequant(w).reshape(N, K).astype(np.float64).T
    assert np.array_equal(got.astype(np.float64), exact)
    want = np.array([[orc.q4k_q8k_vec_dot(K, w[n], x8[t]) for n in range(N)] for t in range(T)], np.float32)
    assert np.array_equal(got, want)


def _cos_rows(a, b):
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


@pytest.mark.parametrize("layout,cfg_name", [("hybrid", "small"), ("q4k", "small"), ("hybrid", "xtr")])
def test_hybrid_forward_vs_oracle_hybrid_variant(enc, layout, cfg_name):
    cfg = synth.small_config() if cfg_name == "small" else dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=64, layout=layout)
    gpu = enc.T5EncoderModel.from_gguf(img, cfg)
    try:
        gpu.set_numerics(1)
        ora = orc.OracleModel(img, cfg, variant=orc.VARIANT_HYBRID)
        ora_default = orc.OracleModel(img, cfg)
        lens = [40, 7, 130] if cfg_name == "small" else [96, 33]
        cu = np.zeros(len(lens) + 1, np.int32)
        cu[1:] = np.cumsum(lens)
        ids = np.random.default_rng(65).integers(1, cfg["vocab_size"], size=int(cu[-1])).astype(np.uint32)
        out, _ = gpu.encode_packed(ids, cu)
        for b in range(len(lens)):
            s, e = cu[b], cu[b + 1]
            ref = ora.forward(ids[s:e])
            assert _cos_rows(out[s:e], ref).min() >= 0.999, (b, float(_cos_rows(out[s:e], ref).min()))
            # against the default numerics: the reference's own backend-comparison bar
            # (tools/compare-backends/src/main.rs:446, cosine >= 0.99)
            assert _cos_rows(out[s:e], ora_default.forward(ids[s:e])).min() >= 0.99
        # query-sized batch (the small-token GEMV kernels around the hybrid FFN)
        q = ids[:32]
        qo, _ = gpu.encode_packed(q, np.array([0, 32], np.int32))
        assert _cos_rows(qo, ora.forward(q)).min() >= 0.999
        # back to the default numerics on the same handle
        gpu.set_numerics(0)
        d, _ = gpu.encode_packed(q, np.array([0, 32], np.int32))
        assert _cos_rows(d, ora_default.forward(q)).min() >= 0.999
    finally:
        gpu.close()


def test_hybrid_layer_teacher_forced(enc):
    """One T5Block with the hybrid FFN against the oracle's hybrid block on the same input:
    relative error <= 1e-3."""
    cfg = dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=64, layout="hybrid")
    gpu = enc.T5EncoderModel.from_gguf(img, cfg)
    try:
        gpu.set_numerics(1)
        ora = orc.OracleModel(img, cfg, variant=orc.VARIANT_HYBRID)
        ids = np.random.default_rng(66).integers(1, cfg["vocab_size"], size=120).astype(np.uint32)
        for layer in (0, 6, 11):
            x = ora.hidden(ids, layer)
            got = gpu.layer_forward(layer, x, np.array([0, 120], np.int32))
            want = ora.layer(layer, x)
            rel = np.linalg.norm(got - want) / np.linalg.norm(want)
            assert rel <= 1e-3, (layer, rel)
    finally:
        gpu.close()


def test_hybrid_ffn_block_pins_the_q8k_numerics(enc):
    """The FFN alone on the same normalised input: the GPU's hybrid FFN is within 1e-3 of the
    oracle's hybrid FFN and clearly closer to it than to the default (f32-activation) FFN,
    whose difference is the Q8_K quantization of the activations."""
    cfg = dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=68)
    gpu = enc.T5EncoderModel.from_gguf(img, cfg)
    try:
        gpu.set_numerics(1)
        ora_h = orc.OracleModel(img, cfg, variant=orc.VARIANT_HYBRID)
        ora_d = orc.OracleModel(img, cfg)
        x = np.random.default_rng(69).standard_normal((96, cfg["d_model"])).astype(np.float32)
        for mode in (0, 1):  # GEMV kernels for wo at T <= 64 do not apply at T = 96; both modes batched
            got = gpu.ffn_block(3, x, mode)
            rel_h = np.linalg.norm(got - ora_h.ffn(3, x)) / np.linalg.norm(ora_h.ffn(3, x))
            rel_d = np.linalg.norm(got - ora_d.ffn(3, x)) / np.linalg.norm(ora_d.ffn(3, x))
            assert rel_h <= 1e-3, (mode, rel_h)
            assert rel_h < 0.25 * rel_d, (mode, rel_h, rel_d)
    finally:
        gpu.close()


def test_set_numerics_rejects_non_q4k_ffn(enc):
    from witchcraft_amd._lib import T5HError
    cfg = synth.small_config()
    # the projection stored F32: the hybrid feature needs it Q4_K (QTiledOp)
    from witchcraft_amd import gguf
    img = synth.make_model(cfg, seed=67)
    ts = gguf.read_gguf(img)
    name = "linear.weight"
    wf = orc.q4k_dequant(np.frombuffer(ts[name].data, np.uint8)).astype(np.float32)
    ts[name] = gguf.Tensor(name, gguf.GGML_F32, ts[name].shape, wf.tobytes())
    gpu = enc.T5EncoderModel.from_gguf(gguf.write_gguf(list(ts.values())), cfg)
    try:
        with pytest.raises(T5HError, match="Q4_K"):
            gpu.set_numerics(1)
        with pytest.raises(T5HError):
            gpu.set_numerics(7)
    finally:
        gpu.close()


def test_q4k_q8k_matmul_multi_tile_vs_oracle(enc):
    """The matrix-core product over several token tiles and a thin tail (T = 300) and 512 weight
    rows, against the oracle's vec_dot per (row, token) within 1e-6 of sum |terms|."""
    rng = np.random.default_rng(70)
    K, N, T = 768, 512, 300
    w = quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x8 = enc.q8k_quantize((rng.standard_normal((T, K)) * rng.uniform(0.1, 10.0, (T, 1))).astype(np.float32))
    got = enc.q4k_q8k_matmul(w, x8, K)
    ts = rng.choice(T, 40, replace=False)
    want = np.array([[orc.q4k_q8k_vec_dot(K, w[n], x8[t]) for n in range(N)] for t in ts], np.float32)
    wd = orc.q4k_dequant(w).reshape(N, K).astype(np.float64)
    xd = np.stack([_q8k_dequant(x8[t]) for t in ts])
    scale = np.abs(xd) @ np.abs(wd).T
    assert np.all(np.abs(got[ts] - want) <= 1e-6 * scale + 1e-30)


def test_hybrid_batch_properties(enc):
    """Hybrid numerics on a ragged batch that spans several tile rows of the hybrid GEMM (lengths
    16..512, 20 sequences): finite, deterministic, sequences encoded alone bit-identical to their
    rows in the batch (every tile plan keeps the K order), and sampled sequences against the
    oracle's hybrid variant."""
    cfg = dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=71, layout="hybrid")
    gpu = enc.T5EncoderModel.from_gguf(img, cfg)
    try:
        gpu.set_numerics(1)
        ids, cu = synth.ragged_batch(20, 16, 512, cfg["vocab_size"], seed=72)
        out, _ = gpu.encode_packed(ids, cu)
        assert np.isfinite(out).all()
        out2, _ = gpu.encode_packed(ids, cu)
        assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
        lens = np.diff(cu)
        long = [int(b) for b in np.argsort(-lens)[:3]] + [int(b) for b in np.where(lens > 64)[0][:3]]
        for b in sorted(set(long)):
            s, e = int(cu[b]), int(cu[b + 1])
            alone, _ = gpu.encode_packed(ids[s:e], np.array([0, e - s], np.int32))
            assert np.array_equal(alone.view(np.uint32), out[s:e].view(np.uint32)), (b, e - s)
        ora = orc.OracleModel(img, cfg, variant=orc.VARIANT_HYBRID)
        for b in (int(np.argmax(lens)), int(np.argmin(lens))):
            s, e = int(cu[b]), int(cu[b + 1])
            assert _cos_rows(out[s:e], ora.forward(ids[s:e])).min() >= 0.999, (b, e - s)
    finally:
        gpu.close()


@pytest.mark.parametrize("lens", [[1], [7, 1, 33], [64, 65]])
def test_hybrid_small_batches_vs_oracle(enc, lens):
    """Hybrid numerics at query-sized and tiny batches (one partial tile of the hybrid GEMM; the
    other linears on the GEMV kernels up to 64 tokens) against the oracle's hybrid variant."""
    cfg = synth.small_config()
    img = synth.make_model(cfg, seed=73)
    gpu = enc.T5EncoderModel.from_gguf(img, cfg)
    try:
        gpu.set_numerics(1)
        ora = orc.OracleModel(img, cfg, variant=orc.VARIANT_HYBRID)
        cu = np.zeros(len(lens) + 1, np.int32)
        cu[1:] = np.cumsum(lens)
        ids = np.random.default_rng(74).integers(1, cfg["vocab_size"], size=int(cu[-1])).astype(np.uint32)
        out, _ = gpu.encode_packed(ids, cu)
        for b in range(len(lens)):
            s, e = int(cu[b]), int(cu[b + 1])
            assert _cos_rows(out[s:e], ora.forward(ids[s:e])).min() >= 0.999, (lens, b)
    finally:
        gpu.close()


def test_q4k_q8k_matmul_single_token(enc):
    rng = np.random.default_rng(75)
    K, N = 256, 64
    w = quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x8 = enc.q8k_quantize(rng.standard_normal((1, K)).astype(np.float32))
    got = enc.q4k_q8k_matmul(w, x8, K)
    want = np.array([[orc.q4k_q8k_vec_dot(K, w[n], x8[0]) for n in range(N)]], np.float32)
    wd = orc.q4k_dequant(w).reshape(N, K).astype(np.float64)
    scale = np.abs(_q8k_dequant(x8[0]))[None, :] @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [193, 200, 450])
def test_q4k_q8k_matmul_tile_padding(enc, T):
    """Token counts whose last full tile reaches past roundup(T, 256): the buffers are padded to
    the hybrid tile height, and every row matches the oracle's vec_dot."""
    rng = np.random.default_rng(76 + T)
    K, N = 512, 128
    w = quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x8 = enc.q8k_quantize(rng.standard_normal((T, K)).astype(np.float32))
    got = enc.q4k_q8k_matmul(w, x8, K)
    assert got.shape == (T, N) and np.isfinite(got).all()
    for t in (0, T // 2, T - 1):
        want = np.array([orc.q4k_q8k_vec_dot(K, w[n], x8[t]) for n in range(N)], np.float32)
        wd = orc.q4k_dequant(w).reshape(N, K).astype(np.float64)
        scale = np.abs(_q8k_dequant(x8[t])) @ np.abs(wd).T
        assert np.all(np.abs(got[t] - want) <= 1e-6 * scale + 1e-30)
