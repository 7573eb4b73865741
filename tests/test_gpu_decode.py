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


# ---- packing (exl3_pack_tiles, the metal-pack codec op) ----


def gpu_pack(states_u16: np.ndarray, k: int):
    import torch

    import mlxl3_amd

    t = torch.from_numpy(states_u16.view(np.int16).ravel().copy()).cuda()
    out = mlxl3_amd.pack_tiles(t, k)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("k", range(1, 9))
def test_pack_matches_oracle_and_inverts_decode(k):
    """Pack of random full 16-bit states uses their low k bits (codec.rs:34-38);
    decoding the packed tiles gives back those k bits as the low bits of every
    state."""
    print(f"pack random tiles k={k}", flush=True)
    rng = np.random.default_rng(500 + k)
    states = rng.integers(0, 65536, (777, 256), dtype=np.uint16)
    packed = gpu_pack(states, k)
    assert np.array_equal(packed, oracle.pack(states, k).ravel())
    back, _ = gpu_decode(packed.reshape(-1, 16 * k), k, 0)
    mask = np.uint16((1 << k) - 1)
    assert np.array_equal(back.ravel() & mask, states.ravel() & mask)


@pytest.mark.parametrize("k", range(2, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_pack_quantizer_corpus_on_gpu(golden, k, cb):
    d = golden / "quantizer"
    packed = np.fromfile(d / f"oracle-{k}-{cb}-packed.u16", "<u2")
    states = np.fromfile(d / f"oracle-{k}-{cb}-states.u16", "<u2")
    assert np.array_equal(gpu_pack(states, k), packed)


def test_metal_pack_codec_op():
    from codec_client import run

    rng = np.random.default_rng(9)
    states = rng.integers(0, 65536, 3 * 256, dtype=np.uint16)
    rows = run([{"op": "metal-pack", "k": 3, "data": states.tolist()},
                {"op": "metal-pack", "k": 3, "data": []},
                {"op": "metal-pack", "k": 3, "data": [0] * 255},
                {"op": "metal-pack", "k": 7, "data": states.tolist()},
                {"op": "metal-pack", "k": 0, "data": []}])
    assert rows[0] == {"data": oracle.pack(states, 3).ravel().tolist()}
    assert rows[1] == {"data": []}
    assert "expected whole 256-state tiles" in rows[2]["error"]
    assert rows[3] == {"data": oracle.pack(states, 7).ravel().tolist()}
    assert "K must be in 1..=8, got 0" in rows[4]["error"]
