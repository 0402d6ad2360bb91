"""Gdn2State interchange (gdn2_state_serialize / gdn2_state_deserialize):
the state as safetensors with the reference's field names
(src/module.rs:30-40).  Checked against the `safetensors` package itself
(reading what the library writes, and the library reading what the package
writes), and by continuing a decode from a round-tripped state."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0, mode="chunk")


def _setup(gpu, B=2, T=70, seed=4):
    import torch

    import gdn2_amd as G

    cfg = G.Gdn2Config(**CFG)
    layer = G.GatedDeltaNet2(cfg, seed=11)
    x = torch.from_numpy(np.random.default_rng(seed).standard_normal((B, T + 3, cfg.hidden_size)).astype(np.float32))
    return G, layer, x.to(gpu)


def test_state_bytes_are_safetensors(gpu):
    from safetensors.numpy import load

    G, layer, x = _setup(gpu)
    _, st = layer.forward(x[:, :70])
    data = st.to_bytes()
    got = load(data)
    assert set(got) == {"recurrent", "conv_q", "conv_k", "conv_v"}
    for name in got:
        assert got[name].dtype == np.float32
        assert np.array_equal(got[name], getattr(st, name)), name
    cfg = layer.config
    assert got["recurrent"].shape == (2, cfg.hv, cfg.head_dim, cfg.v_head)
    assert got["conv_v"].shape == (2, 3, cfg.vd)
    import json

    meta = json.loads(data[8:8 + int.from_bytes(data[:8], "little")])["__metadata__"]
    assert meta["format"] == "gdn2_state" and meta["num_v_heads"] == "4" and meta["head_v_dim"] == "128"


def test_round_trip_continues_identically(gpu):
    """A state rebuilt from its bytes decodes exactly like the original."""
    import torch

    G, layer, x = _setup(gpu)
    _, st = layer.forward(x[:, :70])
    st2 = G.Gdn2State.from_bytes(layer, st.to_bytes())
    assert st2.is_some and st2.batch == 2
    outs = [[], []]
    for t in range(70, 73):
        o1, st = layer.forward(x[:, t:t + 1].contiguous(), st)
        o2, st2 = layer.forward(x[:, t:t + 1].contiguous(), st2)
        outs[0].append(o1)
        outs[1].append(o2)
    assert torch.equal(torch.cat(outs[0], 1), torch.cat(outs[1], 1))
    for name in ("recurrent", "conv_q", "conv_k", "conv_v"):
        assert np.array_equal(getattr(st, name), getattr(st2, name)), name


def test_reads_state_written_by_safetensors(gpu):
    from safetensors.numpy import save

    G, layer, x = _setup(gpu)
    cfg = layer.config
    rng = np.random.default_rng(1)
    tensors = {"recurrent": rng.standard_normal((2, cfg.hv, cfg.head_dim, cfg.v_head)).astype(np.float32),
               "conv_q": rng.standard_normal((2, 3, cfg.kd)).astype(np.float32),
               "conv_k": rng.standard_normal((2, 3, cfg.kd)).astype(np.float32),
               "conv_v": rng.standard_normal((2, 3, cfg.vd)).astype(np.float32)}
    st = G.Gdn2State(layer, 2)
    st.load_bytes(save(tensors, metadata={"format": "gdn2_state"}))
    assert st.is_some
    for name, a in tensors.items():
        assert np.array_equal(getattr(st, name), a), name


def test_deserialize_rejects_mismatches(gpu):
    from safetensors.numpy import save

    from gdn2_amd._capi import Gdn2Error

    G, layer, x = _setup(gpu)
    cfg = layer.config
    good = {"recurrent": np.zeros((2, cfg.hv, cfg.head_dim, cfg.v_head), np.float32),
            "conv_q": np.zeros((2, 3, cfg.kd), np.float32), "conv_k": np.zeros((2, 3, cfg.kd), np.float32),
            "conv_v": np.zeros((2, 3, cfg.vd), np.float32)}
    st = G.Gdn2State(layer, 2)
    with pytest.raises(Gdn2Error, match="state is empty"):
        st.to_bytes()
    bad_shape = dict(good, conv_v=np.zeros((2, 3, cfg.kd), np.float32))
    with pytest.raises(Gdn2Error, match="wrong shape"):
        st.load_bytes(save(bad_shape))
    missing = {k: v for k, v in good.items() if k != "conv_k"}
    with pytest.raises(Gdn2Error, match="'conv_k' missing"):
        st.load_bytes(save(missing))
    wrong_dtype = dict(good, conv_q=good["conv_q"].astype(np.float64))
    with pytest.raises(Gdn2Error, match="not F32"):
        st.load_bytes(save(wrong_dtype))
    with pytest.raises(Gdn2Error, match="truncated header|header length"):
        st.load_bytes(b"\x01\x02")
    assert not st.is_some  # nothing was loaded


def _with_header(header: str, data: bytes) -> bytes:
    h = header.encode()
    h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    return len(h).to_bytes(8, "little") + h + data


def test_deserialize_survives_malformed_bytes(gpu):
    """Every truncation is refused; seeded byte flips in the header either
    load (a flip that leaves a valid header) or raise Gdn2Error; metadata
    nested 100000 deep is refused without recursing into it; a header length
    beyond the buffer is refused.  The good bytes still load afterwards."""
    from gdn2_amd._capi import Gdn2Error

    G, layer, x = _setup(gpu)
    _, st = layer.forward(x[:, :70])
    good = st.to_bytes()
    hn = int.from_bytes(good[:8], "little")
    target = G.Gdn2State(layer, 2)
    rng = np.random.default_rng(5)
    cuts = set(rng.integers(0, len(good), 40).tolist()) | {0, 7, 8, 9, 8 + hn - 1, 8 + hn, len(good) - 1}
    for cut in sorted(cuts):
        with pytest.raises(Gdn2Error):
            target.load_bytes(good[:cut])
    for _ in range(300):
        buf = bytearray(good)
        for pos in rng.integers(8, 8 + hn, int(rng.integers(1, 4))):
            buf[int(pos)] = int(rng.integers(0, 256))
        try:
            target.load_bytes(bytes(buf))
        except Gdn2Error:
            pass
    header = good[8:8 + hn].decode().rstrip(" ")
    deep = header.replace('"__metadata__":{', '"__metadata__":{"x":' + "[" * 100000 + "]" * 100000 + ",", 1)
    with pytest.raises(Gdn2Error, match="malformed"):
        target.load_bytes(_with_header(deep, good[8 + hn:]))
    shallow = header.replace('"__metadata__":{', '"__metadata__":{"x":' + "[" * 8 + "]" * 8 + ",", 1)
    target.load_bytes(_with_header(shallow, good[8 + hn:]))  # moderate nesting is fine
    with pytest.raises(Gdn2Error, match="header length"):
        target.load_bytes((2 ** 63).to_bytes(8, "little") + good[8:])
    target.load_bytes(good)
    for name in ("recurrent", "conv_q", "conv_k", "conv_v"):
        assert np.array_equal(getattr(target, name), getattr(st, name)), name
