"""t5h_encode_device_noalloc through the C ABI against t5h_encode_device on the same handle.

The no-alloc entry point runs the same kernels on a workspace carved from the library's fixed
per-GPU scratch array, so its results must be bit-identical to t5h_encode_device's.  Two calls
in a row, the second on a smaller batch (the array keeps the first call's contents), then a
query-sized batch (the small-token GEMV kernels), then an input whose workspace does not fit.
"""
import numpy as np
import pytest

from witchcraft_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def xtr():
    from witchcraft_amd.encoder import T5EncoderModel
    cfg = dict(synth.XTR_BASE)
    gpu = T5EncoderModel.from_gguf(synth.make_model(cfg, seed=0), cfg)
    yield cfg, gpu
    gpu.close()


def _encode(gpu, noalloc: bool, ids: np.ndarray, cu: np.ndarray):
    import torch
    dev = torch.device("cuda:0")
    T = int(cu[-1])
    d_ids = torch.from_numpy(ids.astype(np.int32)).to(dev)
    d_out = torch.full((T, 128), float("nan"), device=dev)
    d_norm = torch.full((T,), float("nan"), device=dev)
    torch.cuda.synchronize()
    fn = gpu.encode_device_noalloc if noalloc else gpu.encode_device
    fn(d_ids.data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())
    gpu.synchronize()
    return d_out.cpu().numpy(), d_norm.cpu().numpy()


def _batch(cfg, lens, seed):
    cu = np.zeros(len(lens) + 1, np.int32)
    cu[1:] = np.cumsum(lens)
    ids = np.random.default_rng(seed).integers(1, cfg["vocab_size"], size=int(cu[-1])).astype(np.uint32)
    return ids, cu


def test_noalloc_matches_encode_device_twice(xtr):
    cfg, gpu = xtr
    # a larger batch first, then a smaller one, then a query: each call leaves the scratch
    # array holding its own rows, which the next call must not depend on
    for lens, seed in (([300, 77, 512, 129, 65, 256, 200, 1], 1), ([90, 41, 64], 2), ([32], 3)):
        ids, cu = _batch(cfg, lens, seed)
        print(f"[no_alloc] lens={lens}", flush=True)
        ref, nref = _encode(gpu, False, ids, cu)
        got, ngot = _encode(gpu, True, ids, cu)
        assert np.isfinite(ref).all()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), lens
        assert np.array_equal(ngot.view(np.uint32), nref.view(np.uint32)), lens


def test_noalloc_rejects_oversized_input(xtr):
    from witchcraft_amd._lib import T5H_ERR_INVALID, T5HError
    cfg, gpu = xtr
    ids, cu = _batch(cfg, [2048, 2048, 2048], 4)
    with pytest.raises(T5HError) as e:
        _encode(gpu, True, ids, cu)
    assert e.value.code == T5H_ERR_INVALID
    assert "scratch" in str(e.value)
    # the handle and the scratch array still serve a call that fits
    ids, cu = _batch(cfg, [100, 20], 5)
    ref, _ = _encode(gpu, False, ids, cu)
    got, _ = _encode(gpu, True, ids, cu)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_two_handles_back_to_back(xtr):
    """Two handles on one GPU share the scratch array.  Calls from both, enqueued back to back on
    their own streams without any synchronisation between them, must each give the bits of the
    same calls run one at a time: the library chains the calls through a per-GPU event."""
    import torch
    from witchcraft_amd.encoder import T5EncoderModel
    cfg, gpu = xtr
    other = T5EncoderModel.from_gguf(synth.make_model(cfg, seed=0), cfg)
    try:
        dev = torch.device("cuda:0")
        jobs = [(gpu, *_batch(cfg, [400, 300, 211], 11)), (other, *_batch(cfg, [512, 97], 12)),
                (gpu, *_batch(cfg, [90, 41], 13)), (other, *_batch(cfg, [256, 256, 256], 14))]
        refs = [_encode(h, False, ids, cu) for h, ids, cu in jobs]
        bufs = []
        for h, ids, cu in jobs:
            T = int(cu[-1])
            d_ids = torch.from_numpy(ids.astype(np.int32)).to(dev)
            bufs.append((d_ids, torch.full((T, 128), float("nan"), device=dev), torch.full((T,), float("nan"), device=dev)))
        torch.cuda.synchronize()
        for rep in range(3):
            for (h, ids, cu), (d_ids, d_out, d_norm) in zip(jobs, bufs):
                h.encode_device_noalloc(d_ids.data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())
            for h in (gpu, other):
                h.synchronize()
            for k, ((ref, nref), (_, d_out, d_norm)) in enumerate(zip(refs, bufs)):
                got, ngot = d_out.cpu().numpy(), d_norm.cpu().numpy()
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, k)
                assert np.array_equal(ngot.view(np.uint32), nref.view(np.uint32)), (rep, k)
                d_out.fill_(float("nan"))
                d_norm.fill_(float("nan"))
            torch.cuda.synchronize()
    finally:
        other.close()
