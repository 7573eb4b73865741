"""GPU decode through the C ABI (exl3_decode_tiles), bit-exact against the
oracle, the reference's golden vectors, and exhaustively over all 65536 states
of each codebook.  The decode hook runs the same window/decode code as the
QMV and QMM kernels."""

import json

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def gpu_decode(packed_u16: np.ndarray, k: int, cb: int):
    import torch

    import mlxl3_amd

    t = torch.from_numpy(packed_u16.view(np.int16).ravel().copy()).cuda()
    states, values = mlxl3_amd.decode_tiles(t, k, cb)
    torch.cuda.synchronize()
    return states.cpu().numpy().view(np.uint16), values.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("k", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_random_tiles_bit_exact(k, cb):
    print(f"decode random tiles k={k} cb={cb}", flush=True)
    rng = np.random.default_rng(100 * k + cb)
    packed = rng.integers(0, 65536, (1531, 16 * k), dtype=np.uint16)  # odd tile count
    states, values = gpu_decode(packed, k, cb)
    ref_states = oracle.unpack(packed, k)
    assert np.array_equal(states, ref_states)
    assert np.array_equal(values, oracle.codebook(cb)[ref_states])


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_every_state_of_every_codebook(cb):
    """8192 random K=8 tiles cover all 65536 states; every value matches."""
    print(f"decode exhaustive cb={cb}", flush=True)
    rng = np.random.default_rng(7 + cb)
    packed = rng.integers(0, 65536, (8192, 128), dtype=np.uint16)
    states, values = gpu_decode(packed, 8, cb)
    assert np.unique(states).size == 65536
    assert np.array_equal(values, oracle.codebook(cb)[states])


@pytest.mark.parametrize("k", range(2, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_quantizer_corpus_on_gpu(golden, k, cb):
    d = golden / "quantizer"
    packed = np.fromfile(d / f"oracle-{k}-{cb}-packed.u16", "<u2")
    states = np.fromfile(d / f"oracle-{k}-{cb}-states.u16", "<u2").reshape(-1, 256)
    decoded = np.fromfile(d / f"oracle-{k}-{cb}-decoded.f32", "<f4").reshape(-1, 256)
    s, v = gpu_decode(packed.reshape(-1, 16 * k), k, cb)
    assert np.array_equal(s, states)
    got = v.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), decoded.view(np.uint32))


@pytest.mark.parametrize("name", ["flash", "qwen-dense", "qwen-moe", "lfm-moe"])
def test_real_tiles_on_gpu(golden, name):
    fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
    k, cb = fix["k"], fix["mode"]
    packed = np.asarray([t["packed"] for t in fix["tiles"]], np.uint16)
    s, v = gpu_decode(packed, k, cb)
    assert np.array_equal(s, np.asarray([t["states"] for t in fix["tiles"]], np.uint16))
    assert np.array_equal(v, np.asarray([t["f16_bits"] for t in fix["tiles"]], np.uint16))
