"""CPU tests that pin the decoder oracle (oracle/decoder_oracle.c) before it checks the GPU decoder.

Each function is checked against something other than its own formula: closed forms of RoPE and
YaRN (plain RoPE for factor <= 1, the ramp's two ends, the rotation's norm, complex
multiplication), softmax-with-sink closed forms and float64 brute force, the reference's own
invariants (windowed attention equals full attention when the window covers the cache,
src tests/attention_mqa_streaming_tests.rs:16-61), key-order invariance, and an independent
float64 numpy restatement of a whole multi-step decode with cache eviction (the MoE layer there
is the MoE oracle, pinned in tests/test_oracle.py).
"""
import math

import numpy as np
import pytest


def dec():
    from burnext_amd import decoder as D
    return D


# ---------------------------------------------------------------------------------------------
# RoPE / YaRN (src/rope/mod.rs:11-52 over Burn RotaryEncoding)
# ---------------------------------------------------------------------------------------------
def test_rope_plain_frequencies(oracle):
    for d, theta in ((64, 150000.0), (16, 10000.0), (128, 500000.0)):
        inv, conc = oracle.yarn_inv_freq(d, theta, 1.0)
        expect = np.array([theta ** (-2.0 * i / d) for i in range(d // 2)], np.float64).astype(np.float32)
        assert np.array_equal(inv, expect) and conc == 1.0
        # factor below 1 is plain RoPE too (the reference returns config.init() for factor <= 1)
        inv2, conc2 = oracle.yarn_inv_freq(d, theta, 0.5)
        assert np.array_equal(inv2, expect) and conc2 == 1.0


def test_yarn_ramp_ends_and_concentration(oracle):
    d, theta, f, ctx, a, b = 64, 150000.0, 32.0, 4096.0, 1.0, 32.0
    inv, conc = oracle.yarn_inv_freq(d, theta, f, ctx, a, b)
    base = np.array([np.float32(theta ** (-2.0 * i / d)) for i in range(d // 2)], np.float64)
    low = d * math.log(ctx / (b * 2 * math.pi)) / math.log(theta)
    high = d * math.log(ctx / (a * 2 * math.pi)) / math.log(theta)
    assert 0 < low < high < d - 1
    seen = set()
    for i in range(d // 2):
        if 2 * i <= low - 1e-6:      # ramp 0: fully interpolated
            assert inv[i] == np.float32(base[i] / f)
            seen.add("lo")
        elif 2 * i >= high + 1e-6:   # ramp 1: untouched
            assert inv[i] == np.float32(base[i])
            seen.add("hi")
        else:                        # in between, strictly inside
            assert base[i] / f < inv[i] < base[i]
            r = (2 * i - low) / (high - low)
            assert abs(inv[i] - (base[i] / f * (1 - r) + base[i] * r)) <= 1e-6 * base[i]
            seen.add("mid")
    assert seen == {"lo", "mid", "hi"}
    assert abs(conc - (0.1 * math.log(32.0) + 1.0)) < 1e-7
    with pytest.raises(ValueError):  # beta <= alpha: the reference's assert fires
        oracle.yarn_inv_freq(d, theta, f, ctx, 32.0, 1.0)


def test_rope_table_closed_form(oracle):
    inv, conc = oracle.yarn_inv_freq(64, 150000.0, 32.0)
    tab = oracle.rope_table(inv, 64, conc, 300)
    p = np.arange(300, dtype=np.float32)[:, None]
    ang = (p * inv[None, :]).astype(np.float64)  # one f32 product
    assert np.allclose(tab[..., 0], np.cos(ang) * conc, rtol=0, atol=2e-7)
    assert np.allclose(tab[..., 1], np.sin(ang) * conc, rtol=0, atol=2e-7)
    assert np.allclose(np.hypot(tab[..., 0], tab[..., 1]), conc, atol=4e-7)
    assert np.all(tab[0, :, 0] == np.float32(conc)) and np.all(tab[0, :, 1] == 0.0)


def test_rope_apply_is_complex_multiplication(oracle):
    rng = np.random.default_rng(1)
    inv, conc = oracle.yarn_inv_freq(32, 150000.0, 32.0, beta=32.0)
    tab = oracle.rope_table(inv, 32, conc, 64)
    x = rng.standard_normal((5, 32)).astype(np.float32)
    for pos0, stride in ((0, 0), (7, 0), (7, 1), (20, 1)):
        y = oracle.rope_apply(x, pos0, stride, tab)
        for h in range(5):
            p = pos0 + h * stride
            z = (x[h, 0::2] + 1j * x[h, 1::2]).astype(np.complex128) * (tab[p, :, 0] + 1j * tab[p, :, 1])
            assert np.allclose(y[h, 0::2], z.real, atol=1e-6) and np.allclose(y[h, 1::2], z.imag, atol=1e-6)
            assert np.allclose(np.linalg.norm(y[h]), conc * np.linalg.norm(x[h]), rtol=1e-5)
    # head stride 1 rotates head h at pos0 + h: head 0 alike, the others not
    y0, y1 = oracle.rope_apply(x, 3, 0, tab), oracle.rope_apply(x, 3, 1, tab)
    assert np.array_equal(y0[0], y1[0]) and not np.allclose(y0[1:], y1[1:])


# ---------------------------------------------------------------------------------------------
# attention with sinks (src/attention/core.rs:34-55)
# ---------------------------------------------------------------------------------------------
def _attn_f64(q, k, v, nkv, sinks, scale_dk):
    nh, d = q.shape
    g = nh // nkv
    out = np.zeros((nh, d))
    for h in range(nh):
        s = k[:, h // g, :].astype(np.float64) @ q[h].astype(np.float64) / math.sqrt(scale_dk)
        if sinks is not None:
            s = np.append(s, float(sinks[h]))
        e = np.exp(s - s.max())
        w = (e / e.sum())[: k.shape[0]]
        out[h] = w @ v[:, h // g, :].astype(np.float64)
    return out


@pytest.mark.parametrize("nk,nh,nkv,d,sink", [(1, 4, 2, 8, True), (7, 8, 2, 16, True), (33, 4, 4, 8, False),
                                              (64, 16, 2, 64, True)])
def test_sink_attention_vs_f64(oracle, nk, nh, nkv, d, sink):
    rng = np.random.default_rng(nk)
    q = rng.standard_normal((nh, d)).astype(np.float32)
    k = rng.standard_normal((nk, nkv, d)).astype(np.float32) * 0.5
    v = rng.standard_normal((nk, nkv, d)).astype(np.float32)
    s = rng.standard_normal(nh).astype(np.float32) if sink else None
    for scale in (1.0, float(d)):
        got = oracle.sink_attention(q, k, v, nkv, s, scale)
        assert np.allclose(got, _attn_f64(q, k, v, nkv, s, scale), atol=2e-6, rtol=1e-5)


def test_sink_closed_forms(oracle):
    rng = np.random.default_rng(3)
    nh, nkv, d, nk = 4, 2, 8, 5
    q = rng.standard_normal((nh, d)).astype(np.float32)
    k = rng.standard_normal((nk, nkv, d)).astype(np.float32)
    v = rng.standard_normal((nk, nkv, d)).astype(np.float32)
    plain = oracle.sink_attention(q, k, v, nkv, None)
    # a sink far below every score is plain softmax
    assert np.allclose(oracle.sink_attention(q, k, v, nkv, np.full(nh, -1e4, np.float32)), plain, atol=1e-7)
    # identical keys: weights uniform over the keys, the sink takes e^s / (e^s + nk e^score)
    kk = np.broadcast_to(k[:1], k.shape).copy()
    s = np.array([0.0, 1.0, -2.0, 3.0], np.float32)
    got = oracle.sink_attention(q, kk, v, nkv, s)
    g = nh // nkv
    for h in range(nh):
        sc = float(q[h].astype(np.float64) @ kk[0, h // g].astype(np.float64))
        share = math.exp(s[h]) / (math.exp(s[h]) + nk * math.exp(sc))
        assert np.allclose(got[h], (1 - share) * v[:, h // g].astype(np.float64).mean(0), atol=2e-6)
    # key order does not matter
    perm = rng.permutation(nk)
    assert np.allclose(oracle.sink_attention(q, k[perm], v[perm], nkv, s), oracle.sink_attention(q, k, v, nkv, s),
                       atol=1e-6)


# ---------------------------------------------------------------------------------------------
# the whole decode step vs an independent float64 restatement
# ---------------------------------------------------------------------------------------------
def tiny_cfg(**kw):
    D = dec()
    base = dict(vocab_size=97, d_model=64, n_layers=3, n_heads=4, head_dim=16, kv_heads=2, ffn_hidden=64,
                num_experts=4, experts_per_token=2, cache_len=6, window_policy="every_other", window=3,
                full_on_even=True, max_seq_len=64, rope_theta=150000.0, rope_scaling_factor=32.0)
    base.update(kw)
    return D.GptOssConfig(**base)


def _rms64(x, g, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g


def _f64_model(oracle, data, batch):
    """A float64 numpy decoder over the same weights: returns step(tokens, pos, window)."""
    cfg = data.cfg
    W = {k: data.f32(k).astype(np.float64) for k in ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv", "wo",
                                                      "bo", "norm_final", "lm_head")}
    sinks = None if data.sinks is None else data.f32("sinks").astype(np.float64)
    dk, nH, kvH = cfg.head_dim, cfg.n_heads, cfg.kv_heads
    # YaRN from its definition, in float64
    i2 = 2.0 * np.arange(dk // 2)
    inv = cfg.rope_theta ** (-i2 / dk)
    f = cfg.rope_scaling_factor
    conc = 1.0
    if f > 1:
        lb = math.log(cfg.rope_theta)
        low = dk * math.log(cfg.rope_initial_context / (cfg.rope_ntk_beta * 2 * math.pi)) / lb
        high = dk * math.log(cfg.rope_initial_context / (cfg.rope_ntk_alpha * 2 * math.pi)) / lb
        r = np.clip((i2 - low) / (high - low), 0, 1)
        inv = inv / f * (1 - r) + inv * r
        conc = 0.1 * math.log(f) + 1

    def rope(x, p0):  # x [heads, dk]
        y = x.copy()
        for h in range(x.shape[0]):
            a = (p0 + h * cfg.rope_head_stride) * inv
            c, s = np.cos(a) * conc, np.sin(a) * conc
            y[h, 0::2] = x[h, 0::2] * c - x[h, 1::2] * s
            y[h, 1::2] = x[h, 1::2] * c + x[h, 0::2] * s
        return y

    cache = [[[] for _ in range(batch)] for _ in range(cfg.n_layers)]  # rows (k [kvH, dk], v)
    g = nH // kvH

    def step(tokens, pos, window=0):
        h = W["tok_emb"][tokens]
        for l in range(cfg.n_layers):
            xn = _rms64(h, W["norm_attn"][l], cfg.rms_eps)
            q = xn @ W["wq"][l].T + W["bq"][l]
            k = xn @ W["wk"][l].T + W["bk"][l]
            v = xn @ W["wv"][l].T + W["bv"][l]
            lw = cfg.layer_window(l, window)
            ctx = np.zeros((batch, nH * dk))
            for b in range(batch):
                rows = cache[l][b]
                rows.append((rope(k[b].reshape(kvH, dk), pos), v[b].reshape(kvH, dk)))
                S = cfg.sink_tokens
                if len(rows) > cfg.cache_len:  # the oldest row after the sink rows leaves
                    rows.pop(min(S, cfg.cache_len - 1))
                n = len(rows)
                act = rows[n - (S + min(lw, n - S)):] if lw else rows
                qb = rope(q[b].reshape(nH, dk), pos)
                for hh in range(nH):
                    sc = np.array([r[0][hh // g] @ qb[hh] for r in act]) / math.sqrt(cfg.scale_dk)
                    if sinks is not None:
                        sc = np.append(sc, sinks[l, hh])
                    e = np.exp(sc - sc.max())
                    wts = (e / e.sum())[: len(act)]
                    ctx[b, hh * dk:(hh + 1) * dk] = sum(wt * r[1][hh // g] for wt, r in zip(wts, act))
            h = h + ctx @ W["wo"][l].T + W["bo"][l]
            h = oracle.moe_forward(data.moe[l], h.astype(np.float32),
                                   bf16_rows=cfg.experts_bf16)[0].astype(np.float64)
        hid = h
        logits = _rms64(h, W["norm_final"], cfg.rms_eps) @ W["lm_head"].T
        return logits, hid

    def load(k, v):  # cache rows [L, B, len, kvH, dk] for positions 0 .. len-1
        for l in range(cfg.n_layers):
            for b in range(batch):
                cache[l][b][:] = [(k[l, b, r].astype(np.float64), v[l, b, r].astype(np.float64))
                                  for r in range(k.shape[2])]

    step.load = load
    return step


@pytest.mark.parametrize("kw,window", [(dict(), 0), (dict(window_policy="fixed", window=4), 0),
                                       (dict(window_policy="full", rope_head_stride=0), 2),
                                       (dict(rope_scaling_factor=1.0, full_on_even=False), 0),
                                       # sink rows kept through eviction; windows widened by them
                                       (dict(sink_tokens=1), 0), (dict(sink_tokens=2, window=2), 0),
                                       (dict(sink_tokens=2, window_policy="full"), 2),
                                       (dict(sink_tokens=5), 0),  # cache_len - 1: nothing rolls
                                       (dict(experts_bf16=True), 0)])  # the MoE layers on bf16 rows
def test_decoder_step_vs_f64(oracle, kw, window):
    D = dec()
    cfg = tiny_cfg(**kw)
    data = D.make_decoder(cfg, seed=5, sinks_std=0.7, norm_std=0.1, moe_dtype="f32")
    B = 2
    orc = oracle.DecoderOracle(data, B)
    ref = _f64_model(oracle, data, B)
    rng = np.random.default_rng(0)
    S = cfg.sink_tokens
    if S:  # a windowed layer needs the sink rows in the cache: load them (what a prefill leaves)
        shape = (cfg.n_layers, B, S, cfg.kv_heads, cfg.head_dim)
        k, v = rng.standard_normal(shape).astype(np.float32), rng.standard_normal(shape).astype(np.float32)
        orc.load(k, v)
        ref.load(k, v)
    for pos in range(S, S + 10):  # cache_len 6: positions 6.. evict
        tok = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
        nxt, lg, hid = orc.step(tok, pos, window)
        lg64, hid64 = ref(tok, pos, window)
        assert oracle.max_abs_rel(hid, hid64) < 2e-5, pos
        assert oracle.max_abs_rel(lg, lg64) < 2e-5, pos
        top2 = np.sort(lg64, axis=1)[:, -2:]
        for b in range(B):
            if top2[b, 1] - top2[b, 0] > 1e-4 * np.abs(lg64).max():
                assert nxt[b] == int(np.argmax(lg64[b])), (pos, b)
    assert orc.used == cfg.cache_len


def test_sink_rows_survive_eviction(oracle):
    """With sink_tokens S the first S cache rows are the first S positions' rows after any number of
    evictions (src/attention/cache_ops.rs:64-117), and the other rows are the latest positions in
    order; without sinks the cache is the latest cache_len positions."""
    D = dec()
    for S in (0, 2, 5):
        cfg = tiny_cfg(sink_tokens=S, window_policy="full")
        data = D.make_decoder(cfg, seed=4, moe_dtype="f32")
        orc = oracle.DecoderOracle(data, 1)
        rows = {}
        for pos in range(15):
            orc.step(np.array([pos % cfg.vocab_size], np.int32), pos)
            rows[pos] = orc.k[0, 0, min(pos, cfg.cache_len - 1)].copy()  # the row a step appends
        cap = cfg.cache_len
        expect = list(range(S)) + list(range(15 - (cap - S), 15))
        for r, p in enumerate(expect):
            assert np.array_equal(orc.k[0, 0, r], rows[p]), (S, r, p)


def test_window_with_too_few_sink_rows_is_refused(oracle):
    """A windowed layer over fewer cache rows than sink_tokens has no window in the reference (its
    gathered rows and the window length disagree): the oracle refuses the step."""
    D = dec()
    cfg = tiny_cfg(sink_tokens=3)
    data = D.make_decoder(cfg, seed=4, moe_dtype="f32")
    orc = oracle.DecoderOracle(data, 1)
    with pytest.raises(AssertionError):
        orc.step(np.array([1], np.int32), 0)


def test_window_covering_cache_equals_full(oracle):
    """The reference's streaming_mqa_window_matches_full, for the decode step: a caller window that
    covers every cached row gives the same step as Full, bit for bit."""
    D = dec()
    cfg = tiny_cfg(window_policy="full", cache_len=8)
    data = D.make_decoder(cfg, seed=2, sinks_std=0.5, moe_dtype="f32")
    a, b = oracle.DecoderOracle(data, 1), oracle.DecoderOracle(data, 1)
    for pos in range(6):
        tok = np.array([pos * 7 % cfg.vocab_size], np.int32)
        ra, rb = a.step(tok, pos, 0), b.step(tok, pos, 8)
        for x, y in zip(ra, rb):
            assert np.array_equal(x, y)


def test_cache_load_equals_decoded_prefix(oracle):
    """Loading the cache rows a decode wrote reproduces the next step exactly."""
    D = dec()
    cfg = tiny_cfg(cache_len=8)
    data = D.make_decoder(cfg, seed=3, sinks_std=0.5, moe_dtype="f32")
    a = oracle.DecoderOracle(data, 2)
    for pos in range(4):
        a.step(np.array([pos, pos + 1], np.int32), pos)
    b = oracle.DecoderOracle(data, 2)
    b.load(a.k[:, :, :4].copy(), a.v[:, :, :4].copy())
    ra = a.step(np.array([9, 11], np.int32), 4)
    rb = b.step(np.array([9, 11], np.int32), 4)
    for x, y in zip(ra, rb):
        assert np.array_equal(x, y)
