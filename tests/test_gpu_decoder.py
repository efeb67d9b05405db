"""GPU parity of the decoder decode step (include/burnext_gptoss.h) against the CPU decoder oracle.

Bars: with f32 cache rows (the reference's element) logits and the final hidden state within
max|y - y_ref| / max|y_ref| <= 5e-4 of the oracle at every step, greedy tokens equal wherever the
oracle's top-2 margin exceeds that tolerance; with bf16 cache rows within the bf16 bar 2e-2.  The
cases cover cache eviction (positions past cache_len), every window policy and the caller's
window, sinks, head-indexed and per-token RoPE positions, YaRN on and off, partial row tiles
(vocabulary not a multiple of 16), group sizes 1..16 and the GPT-OSS-20B shapes with an 8192-row
cache.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL_F32 = 5e-4
TOL_BF16 = 2e-2
# experts_bf16 against the oracle that rounds the same rows: the device's f32 rows and SwiGLU
# outputs differ from the oracle's in the last bits (summation order), so now and then one value
# rounds to the other bf16 neighbour; one such value moves a row by up to a few 1e-3
TOL_EXPERTS_BF16 = 5e-3


@pytest.fixture(scope="module")
def D():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from burnext_amd import decoder
    return decoder


def _np(t):
    return t.detach().float().cpu().numpy()


def _cfg(D, **kw):
    base = dict(vocab_size=509, d_model=256, n_layers=4, n_heads=8, head_dim=32, kv_heads=2, ffn_hidden=256,
                num_experts=4, experts_per_token=2, cache_len=40, window_policy="every_other", window=8,
                full_on_even=True, max_seq_len=128)
    base.update(kw)
    return D.GptOssConfig(**base)


def _check_step(oracle, tol, nxt, lg, hid, o_nxt, o_lg, o_hid, where):
    assert oracle.max_abs_rel(_np(hid), o_hid) <= tol, (where, oracle.max_abs_rel(_np(hid), o_hid))
    assert oracle.max_abs_rel(_np(lg), o_lg) <= tol, (where, oracle.max_abs_rel(_np(lg), o_lg))
    top2 = np.sort(o_lg, axis=1)[:, -2:]
    scale = np.abs(o_lg).max()
    n = _np(nxt).astype(np.int64)
    for b in range(o_lg.shape[0]):
        if top2[b, 1] - top2[b, 0] > 2 * tol * scale:
            assert n[b] == o_nxt[b], (where, b)


CASES = {
    "every_other": dict(),
    "every_other_odd_full": dict(full_on_even=False),
    "fixed": dict(window_policy="fixed", window=5),
    "full_stride0": dict(window_policy="full", rope_head_stride=0),
    "no_yarn_no_sinks": dict(use_ntk_yarn=False, learned_sinks=False),
    "groups1": dict(n_heads=4, kv_heads=4, head_dim=64),
    "groups16": dict(n_heads=16, kv_heads=1, head_dim=16),
    "dk128": dict(n_heads=4, kv_heads=2, head_dim=128, cache_len=300, window=200, max_seq_len=512),
    # the MoE combine that also writes the next norm, over its slot-row layouts: 4 down K-parts
    # (few touched experts, F = 512), unsplit rows (F = 96); d_model 4160 > 4096 keeps the
    # separate rmsnorm_kernel after every MoE layer
    "combine_norm_4parts": dict(ffn_hidden=512),
    "combine_norm_unsplit": dict(ffn_hidden=96),
    "wide_d_unfused": dict(d_model=4160, n_layers=2),
    # an output projection of 32 K-parts (512 rows x 4096 inputs: few row tiles, so 4 K-groups per
    # part), more than the router that forms the residual row takes: the separate residual add
    "wo_32_parts": dict(d_model=512, n_heads=32, head_dim=128, kv_heads=8, n_layers=2),
}


@pytest.mark.parametrize("case", list(CASES))
def test_decode_steps_match_oracle(D, oracle, case):
    """Teacher-forced decode past cache eviction; tokens fed to both sides are the oracle's greedy
    choices, so a near-tie cannot fork the two sequences."""
    cfg = _cfg(D, **CASES[case])
    data = D.make_decoder(cfg, seed=11, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B = 3
    print(f"[decoder] case={case} cfg={cfg}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=B)
    orc = oracle.DecoderOracle(data, B)
    rng = np.random.default_rng(7)
    tok = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
    caller = 6 if case == "full_stride0" else 0
    steps = cfg.cache_len + 12
    for pos in range(steps):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True, window=caller)
        o_nxt, o_lg, o_hid = orc.step(tok, pos, caller)
        torch.cuda.synchronize()
        _check_step(oracle, TOL_F32, nxt, lg, hid, o_nxt, o_lg, o_hid, (case, pos))
        tok = o_nxt
    dev.close()


@pytest.mark.parametrize("kw", [dict(), dict(window_policy="full", cache_len=300, max_seq_len=700),
                                dict(experts_bf16=True)])
def test_decode_batch1_matches_oracle(D, oracle, kw):
    """Batch-1 decoding: each MoE layer sees a single token, which routes inside its gate_up launch
    (the top K picked by every workgroup, the records and routing outputs written there) after the
    router that forms the residual row.  Teacher-forced past cache eviction (two key chunks in the
    full-window case) against the decoder oracle (with the bf16 rows modelled for experts_bf16, four
    steps: see test_decode_experts_bf16)."""
    cfg = _cfg(D, **kw)
    data = D.make_decoder(cfg, seed=16, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    print(f"[decoder] batch 1 {kw}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=1)
    orc = oracle.DecoderOracle(data, 1)
    tok = np.array([57], np.int32)
    bf = cfg.experts_bf16
    steps = 4 if bf else cfg.cache_len + 12
    for pos in range(steps):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        torch.cuda.synchronize()
        _check_step(oracle, TOL_EXPERTS_BF16 if bf else TOL_F32, nxt, lg, hid, o_nxt, o_lg, o_hid, (kw, pos))
        tok = o_nxt
    dev.close()


@pytest.mark.parametrize("kw,caller", [
    (dict(sink_tokens=4), 0),                                       # every-other 8-row windows
    (dict(sink_tokens=3, window_policy="fixed", window=5), 0),
    (dict(sink_tokens=2, window_policy="full", cache_len=300, max_seq_len=700), 0),  # two key chunks
    (dict(sink_tokens=39, window_policy="full"), 6),                # one non-sink row: nothing rolls
])
def test_decode_sink_tokens(D, oracle, kw, caller):
    """GptOssConfig.sink_tokens: the cache keeps the first positions' rows through eviction and
    windows span the last sink + min(w, rows - sink) rows (src/attention/cache_ops.rs:64-117,
    src/attention/streaming_mqa.rs:332-339).  The sink rows are loaded first (a windowed layer needs
    them), then teacher-forced steps past several evictions."""
    cfg = _cfg(D, **kw)
    data = D.make_decoder(cfg, seed=14, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B, S = 3, cfg.sink_tokens
    print(f"[decoder] sink_tokens cfg={cfg}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=B)
    from burnext_amd import _native as N
    if cfg.window_policy != "full" or caller:
        with pytest.raises(N.BurnextError, match="sink_tokens"):  # no sink rows yet
            dev.decode(torch.zeros(B, dtype=torch.int32, device="cuda"), 0, window=caller)
    orc = oracle.DecoderOracle(data, B)
    rng = np.random.default_rng(8)
    shape = (cfg.n_layers, B, S, cfg.kv_heads, cfg.head_dim)
    k = (rng.standard_normal(shape, dtype=np.float32) * 0.6).astype(np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    dev.cache_load(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    orc.load(k, v)
    tok = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
    steps = cfg.cache_len + 12 if cfg.cache_len < 100 else 2 * cfg.cache_len - 2 * S + 5
    for pos in range(S, S + steps):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True, window=caller)
        o_nxt, o_lg, o_hid = orc.step(tok, pos, caller)
        torch.cuda.synchronize()
        _check_step(oracle, TOL_F32, nxt, lg, hid, o_nxt, o_lg, o_hid, (kw, pos))
        tok = o_nxt
    dev.close()


@pytest.mark.parametrize("vocab,B", [(1000, 1), (1000, 5), (1000, 8), (4099, 3), (1000, 12), (509, 16)])
def test_decode_lm_head_paths(D, oracle, vocab, B):
    """The LM head's two paths against the oracle's logits and greedy tokens: batches of at most 8
    rows stream the matrix in equal runs of K-groups, one per wave (vocabularies of 1000 and 4099
    rows: runs that cut row tiles, whose two parts the fix-up kernel adds, and a last tile of 8 or 3
    rows); 12 and 16 rows take the K-split GEMV and the logits kernel."""
    cfg = _cfg(D, vocab_size=vocab)
    data = D.make_decoder(cfg, seed=17, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    print(f"[decoder] LM head vocab={vocab} B={B}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=B)
    orc = oracle.DecoderOracle(data, B)
    rng = np.random.default_rng(3)
    tok = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
    for pos in range(4):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        torch.cuda.synchronize()
        _check_step(oracle, TOL_F32, nxt, lg, hid, o_nxt, o_lg, o_hid, (vocab, B, pos))
        tok = o_nxt
    dev.close()


def test_decode_bf16_cache(D, oracle):
    cfg = _cfg(D, kv_bf16=True)
    data = D.make_decoder(cfg, seed=12, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B = 2
    dev = D.GptOssDecoder(data, max_batch=B)
    orc = oracle.DecoderOracle(data, B)
    tok = np.array([3, 100], np.int32)
    for pos in range(cfg.cache_len + 5):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        _check_step(oracle, TOL_BF16, nxt, lg, hid, o_nxt, o_lg, o_hid, pos)
        tok = o_nxt


@pytest.mark.parametrize("case", ["every_other", "wo_32_parts", "wide_d_unfused", "groups16"])
def test_decode_experts_bf16(D, oracle, case):
    """experts_bf16 (the expert projections on bf16-rounded rows) against the oracle that rounds the
    same rows (its bf16_rows mode), four steps.  The cases take the router that also forms the
    residual row, the separate residual add with the decode router, and (d_model 4160) the
    general router.  (Over many steps a value rounded to the other bf16 neighbour can move a
    later layer's expert choice: the single-layer test below runs the whole eviction range.)"""
    cfg = _cfg(D, experts_bf16=True, **CASES[case])
    data = D.make_decoder(cfg, seed=14, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B = 3
    print(f"[decoder] experts_bf16 {case}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=B)
    orc = oracle.DecoderOracle(data, B)
    tok = np.array([3, 100, 7], np.int32)
    for pos in range(4):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        _check_step(oracle, TOL_EXPERTS_BF16, nxt, lg, hid, o_nxt, o_lg, o_hid, (case, pos))
        tok = o_nxt
    dev.close()


def test_decode_experts_bf16_vs_f32(D, oracle):
    """experts_bf16 against the f32 decoder oracle (the reference's arithmetic) within the bf16 bar,
    one layer over the whole eviction range (its cache rows come from the embeddings alone, so
    they stay equal to the oracle's)."""
    cfg = _cfg(D, experts_bf16=True, n_layers=1)
    data = D.make_decoder(cfg, seed=15, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B = 4
    dev = D.GptOssDecoder(data, max_batch=B)
    orc = oracle.DecoderOracle(data, B, experts_bf16=False)
    tok = np.array([3, 100, 7, 250], np.int32)
    for pos in range(cfg.cache_len + 3):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        _check_step(oracle, TOL_BF16, nxt, lg, hid, o_nxt, o_lg, o_hid, pos)
        tok = o_nxt
    dev.close()


def test_greedy_generation_and_null_outputs(D, oracle):
    """Free-running greedy generation equals the oracle's token for token; the step without
    logits / hidden outputs returns the same tokens; batch rows are independent."""
    cfg = _cfg(D, cache_len=24)
    data = D.make_decoder(cfg, seed=13, sinks_std=0.8, norm_std=0.1, moe_dtype="f32")
    B = 4
    first = np.array([1, 2, 3, 1], np.int32)
    dev = D.GptOssDecoder(data, max_batch=B)
    gen = _np(dev.generate(torch.from_numpy(first).cuda(), 0, 30)).astype(np.int32)
    orc = oracle.DecoderOracle(data, B)
    tok, seq = first, []
    for pos in range(30):
        tok, _, _ = orc.step(tok, pos)
        seq.append(tok)
    assert np.array_equal(gen, np.stack(seq, 1))
    assert np.array_equal(gen[0], gen[3])  # identical prompts, identical rows
    dev.reset()
    out = dev.decode(torch.from_numpy(first).cuda(), 0)
    assert np.array_equal(_np(out).astype(np.int32), gen[:, 0])
    # a smaller batch on the same decoder
    dev.reset()
    out2 = dev.decode(torch.from_numpy(first[:1]).cuda(), 0)
    assert int(_np(out2)[0]) == gen[0, 0]


def test_decode_argument_errors(D):
    from burnext_amd import _native as N
    cfg = _cfg(D, n_layers=2, max_seq_len=8)
    data = D.make_decoder(cfg, seed=1, moe_dtype="f32")
    dev = D.GptOssDecoder(data, max_batch=2)
    tok = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(N.BurnextError, match="not the next position"):
        dev.decode(tok, 3)
    with pytest.raises(N.BurnextError, match="batch"):
        dev.decode(torch.zeros(3, dtype=torch.int32, device="cuda"), 0)
    ws = dev.workspace(2)
    with pytest.raises(N.BurnextError, match="WORKSPACE_TOO_SMALL"):
        dev.decode(tok, 0, workspace=ws[:ws.numel() // 2])
    # a batch row the cache holds no rows for is refused while the cache is not empty
    dev.decode(tok[:1], 0)
    with pytest.raises(N.BurnextError, match="batch rows the cache holds"):
        dev.decode(tok, 1)
    dev.reset()
    for p in range(8):
        dev.decode(tok, p)
    with pytest.raises(N.BurnextError, match="max_positions"):
        dev.decode(tok, 8)
    dev.reset()
    k = torch.zeros((2, 1, 3, cfg.kv_heads, cfg.head_dim), device="cuda")
    dev.cache_load(k, k)  # 3 rows for batch row 0 only
    with pytest.raises(N.BurnextError, match="batch rows the cache holds"):
        dev.decode(tok, 3)
    dev.decode(tok[:1], 3)
    torch.cuda.synchronize()


def test_decode_c5_full_size(D, oracle):
    """The benchmark's C5 decoder itself (24 layers, d_model 2880, 64 q / 8 kv heads of 64,
    alternating 128-row window and full layers with learned sinks, YaRN factor 32 base 150000,
    vocabulary 201088, 32 experts top-4, f32 cache of 8192 rows, batch 8; the bench's weights,
    seed 0): the cache loaded with 8191 rows, two greedy steps -- the first fills the cache, the
    second evicts its oldest row -- against the decoder oracle's logits, hidden state and tokens."""
    cfg = D.GptOssConfig(max_seq_len=8192 + 64)
    assert (cfg.n_layers, cfg.vocab_size, cfg.cache_len) == (24, 201088, 8192)
    print("[decoder] C5 full size: generating weights", flush=True)
    data = D.make_decoder(cfg, seed=0, sinks_std=0.5)
    B, pre = 8, cfg.cache_len - 1
    rng = np.random.default_rng(7)
    shape = (cfg.n_layers, B, pre, cfg.kv_heads, cfg.head_dim)
    k = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.6)
    v = rng.standard_normal(shape, dtype=np.float32)
    dev = D.GptOssDecoder(data, max_batch=B)
    dev.cache_load(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    orc = oracle.DecoderOracle(data, B)
    orc.load(k, v)
    del k, v
    tok = (np.arange(B, dtype=np.int32) * 1009) % cfg.vocab_size
    for pos in range(pre, pre + 2):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        torch.cuda.synchronize()
        print(f"[decoder] C5 full size: GPU step at pos {pos} done, oracle step", flush=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        print(f"C5 pos {pos}: logits max-abs-rel {oracle.max_abs_rel(_np(lg), o_lg):.3e}, hidden "
              f"{oracle.max_abs_rel(_np(hid), o_hid):.3e}, tokens {_np(nxt).astype(int).tolist()} / {o_nxt.tolist()}",
              flush=True)
        _check_step(oracle, TOL_F32, nxt, lg, hid, o_nxt, o_lg, o_hid, pos)
        tok = o_nxt
    dev.close()


@pytest.mark.parametrize("kv_bf16,experts_bf16", [(False, False), (True, False), (False, True)])
def test_decode_20b_shapes_full_cache(D, oracle, kv_bf16, experts_bf16):
    """GPT-OSS-20B layer shapes (d_model 2880, 64 q / 8 kv heads of 64, 32 experts top-4, 128-row
    window on the odd layer) with an 8192-row cache loaded to 8190 rows: three steps fill it and
    evict the oldest row."""
    cfg = D.GptOssConfig(vocab_size=50001, n_layers=2, kv_bf16=kv_bf16, experts_bf16=experts_bf16, max_seq_len=16384)
    data = D.make_decoder(cfg, seed=21, sinks_std=0.8, norm_std=0.1)
    B, pre = 8, cfg.cache_len - 2
    rng = np.random.default_rng(5)
    shape = (cfg.n_layers, B, pre, cfg.kv_heads, cfg.head_dim)
    k = (rng.standard_normal(shape, dtype=np.float32) * 0.6).astype(np.float32)
    v = rng.standard_normal(shape, dtype=np.float32).astype(np.float32)
    print(f"[decoder] 20b shapes kv_bf16={kv_bf16} experts_bf16={experts_bf16}", flush=True)
    dev = D.GptOssDecoder(data, max_batch=B)
    dev.cache_load(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    orc = oracle.DecoderOracle(data, B)
    if kv_bf16:
        from burnext_amd.synth import round_bf16
        orc.load(round_bf16(k).reshape(shape), round_bf16(v).reshape(shape))
    else:
        orc.load(k, v)
    del k, v
    tok = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
    # the oracle rounds the expert rows as experts_bf16 does
    tol = TOL_BF16 if kv_bf16 else TOL_EXPERTS_BF16 if experts_bf16 else TOL_F32
    for pos in range(pre, pre + 3):
        nxt, lg, hid = dev.decode(torch.from_numpy(tok).cuda(), pos, logits=True, hidden=True)
        o_nxt, o_lg, o_hid = orc.step(tok, pos)
        _check_step(oracle, tol, nxt, lg, hid, o_nxt, o_lg, o_hid, pos)
        tok = o_nxt
    dev.close()
