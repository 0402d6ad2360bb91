"""Host-side layer logic through the C ABI (include/gdn2_layer.h), no GPU:
Gdn2Config::validate (src/config.rs:71-111), Default (:114-130), the shape
algebra (src/module.rs:113-119), the parameter table and the initialisers of
GatedDeltaNet2::new (src/module.rs:111-190).

burn's RNG stream cannot be reproduced without burn, so the initial values
are pinned by their distributions (bounds, moments, the dt_bias inverse
softplus identity), not by values: the layer parity tests feed the same
weights to the oracle and to the GPU."""
import math

import numpy as np
import pytest

import gdn2_amd as G


def test_default_matches_reference():
    c = G.Gdn2Config()
    c.validate()
    from gdn2_amd import _capi as C
    import ctypes

    d = C.Config()
    C.lib().gdn2_config_default(ctypes.byref(d))
    assert (d.hidden_size, d.num_heads, d.head_dim, d.expand_v, d.num_v_heads) == (2048, 16, 128, 1.0, 0)
    assert (d.use_short_conv, d.allow_neg_eigval, d.norm_eps, d.mode, d.chunk_size, d.has_min_decay) == (
        1, 0, 1e-5, C.MODE_FUSED_RECURRENT, 64, 0)
    assert d.gva_layout == C.GVA_HEAD_REPEAT
    assert c.to_c().hidden_size == d.hidden_size and c.to_c().mode == d.mode
    assert c.to_c().gva_layout == d.gva_layout


def test_gva_layout_is_checked_after_the_reference_checks():
    """gva_layout is this library's field: the C check runs after the
    reference's (an invalid config reports the reference's message first),
    and the Python mirror refuses unknown names."""
    import ctypes

    from gdn2_amd import _capi as C

    d = G.Gdn2Config(num_heads=8, num_v_heads=16, gva_layout="reference").to_c()
    assert C.lib().gdn2_config_validate(ctypes.byref(d)) == C.GDN2_OK
    d.gva_layout = 2
    assert C.lib().gdn2_config_validate(ctypes.byref(d)) == C.GDN2_EINVAL
    assert "gva_layout" in C.lib().gdn2_last_error().decode()
    d.hidden_size = 0
    assert C.lib().gdn2_config_validate(ctypes.byref(d)) == C.GDN2_EINVAL
    assert C.lib().gdn2_last_error().decode().startswith("hidden_size must be > 0")
    with pytest.raises(ValueError):
        G.Gdn2Config(gva_layout="scrambled").to_c()


# (overrides, the reference's panic message) in the order validate checks them
PANICS = [
    (dict(hidden_size=0), "hidden_size must be > 0, got 0"),
    (dict(num_heads=0), "num_heads must be > 0, got 0"),
    (dict(head_dim=0), "head_dim must be > 0, got 0"),
    (dict(expand_v=0.3), "expand_v=0.3 must produce an integer head_v_dim when multiplied by head_dim=128 (got 38.4)"),
    (dict(expand_v=-1.0), "expand_v=-1 must produce an integer head_v_dim"),
    (dict(num_v_heads=8), "num_v_heads=8 < num_heads=16 is not supported; use num_v_heads >= num_heads "
                          "(GVA repeats key-side heads)"),
    (dict(num_v_heads=24), "num_v_heads=24 must be divisible by num_heads=16"),
    (dict(chunk_size=0), "chunk_size must be > 0, got 0"),
    (dict(norm_eps=0.0), "norm_eps must be > 0, got 0"),
]


@pytest.mark.parametrize("over,msg", PANICS, ids=[m.split(" ")[0] for _, m in PANICS])
def test_validate_panics_like_reference(over, msg):
    with pytest.raises(ValueError) as e:
        G.Gdn2Config(**over).validate()
    assert str(e.value).startswith(msg)


def test_validate_accepts_the_benchmark_configs():
    for c in CONFIGS.values():
        c.validate()


CONFIGS = {
    "C1": G.Gdn2Config(hidden_size=256, num_heads=4, head_dim=64, mode="chunk"),
    "C2": G.Gdn2Config(mode="chunk"),
    "C3": G.Gdn2Config(),
    "C4": G.Gdn2Config(num_heads=8, num_v_heads=16, expand_v=2.0, allow_neg_eigval=True, min_decay=0.9, mode="chunk"),
    "C5": G.Gdn2Config(mode="chunk", chunk_size=128),
}


def test_shape_algebra():
    import ctypes

    from gdn2_amd import _capi as C

    expect = {"C1": (4, 64, 256, 256), "C2": (16, 128, 2048, 2048), "C4": (16, 256, 1024, 4096)}
    for name, dims in expect.items():
        c = CONFIGS[name]
        out = [C._i64() for _ in range(4)]
        assert C.lib().gdn2_config_dims(ctypes.byref(c.to_c()), *[ctypes.byref(o) for o in out]) == 0
        assert tuple(o.value for o in out) == dims == (c.hv, c.v_head, c.kd, c.vd)


def test_param_table_and_counts():
    names = G.param_names()
    assert names[:3] == ("q_proj", "k_proj", "v_proj") and names[-1] == "decay_factors" and len(names) == 18
    c2, c4 = CONFIGS["C2"], CONFIGS["C4"]
    assert G.param_shape(c2, "f_proj_0") == (2048, 128) and G.param_shape(c2, "f_proj_1") == (128, 2048)
    assert G.param_shape(c4, "v_proj") == (2048, 4096) and G.param_shape(c4, "o_proj") == (4096, 2048)
    assert G.param_shape(c4, "g_proj_1") == (256, 4096) and G.param_shape(c4, "decay_factors") == (8, 128)
    assert G.param_shape(c2, "decay_factors") == ()
    with pytest.raises(KeyError):
        G.param_shape(c2, "no_such_param")
    n2 = sum(int(np.prod(G.param_shape(c2, n) or (0,))) for n in names)
    n4 = sum(int(np.prod(G.param_shape(c4, n) or (0,))) for n in names)
    assert round(n2 / 1e6, 1) == 26.2 and round(n4 / 1e6, 1) == 33.8


def test_init_distributions():
    c = G.Gdn2Config(hidden_size=512, num_heads=4, head_dim=64, expand_v=2.0, min_decay=0.9)
    p = G.init_params(c, seed=7)
    gain = 2.0 ** -2.5
    for n in ("q_proj", "k_proj", "v_proj", "f_proj_0", "f_proj_1", "b_proj", "w_proj", "g_proj_0", "g_proj_1",
              "o_proj"):
        w = p[n].astype(np.float64)
        bound = gain * math.sqrt(6.0 / sum(w.shape))
        assert np.abs(w).max() <= bound * (1 + 1e-6) and np.abs(w).max() > 0.99 * bound
        assert abs(w.mean()) < 0.02 * bound
        assert abs(w.var() / (bound * bound / 3.0) - 1.0) < 0.05
    assert not np.any(p["g_proj_1_bias"])
    assert np.all(p["o_norm_weight"] == 1.0) and np.all(p["decay_factors"] == 2.0)
    assert p["a_log"].min() >= 0.0 and p["a_log"].max() <= math.log(16.0)
    for n in ("q_conv_w", "k_conv_w", "v_conv_w"):
        assert np.abs(p[n]).max() <= 0.5 and abs(p[n].std() - 1 / math.sqrt(12)) < 0.02
    # dt_bias is the inverse softplus of a log-uniform dt in [1e-3, 0.1]
    dt = np.log1p(np.exp(p["dt_bias"].astype(np.float64)))
    assert dt.min() >= 1e-3 * (1 - 1e-4) and dt.max() <= 0.1 * (1 + 1e-4)
    ld = np.log(dt)
    assert abs(ld.mean() - 0.5 * (math.log(1e-3) + math.log(0.1))) < 0.15
    assert abs(ld.std() - (math.log(0.1) - math.log(1e-3)) / math.sqrt(12)) < 0.1


def test_init_is_seeded_and_streams_are_independent():
    c = G.Gdn2Config(hidden_size=128, num_heads=2, head_dim=64)
    a, b, d = G.init_params(c, 1), G.init_params(c, 1), G.init_params(c, 2)
    for n in a:
        if a[n] is not None:
            assert np.array_equal(a[n], b[n])
    assert not np.array_equal(a["q_proj"], d["q_proj"])
    # two parameters of equal shape are not shifted copies of one stream
    q, k = a["q_proj"].ravel().astype(np.float64), a["k_proj"].ravel().astype(np.float64)
    for s in range(0, 8):
        assert abs(np.corrcoef(q[s:], k[:q.size - s])[0, 1]) < 0.05
        assert abs(np.corrcoef(k[s:], q[:q.size - s])[0, 1]) < 0.05
