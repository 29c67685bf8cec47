"""Whole-step parity of the fused decode engine against the CPU oracle.

Bars (from the task's north star): per-step logits within 1e-4 relative
(max |gpu - cpu| / max |cpu|), greedy tokens identical.  Greedy sequences are
checked teacher-forced: both sides are fed the oracle's token at every step,
so one near-tie cannot derail the rest of the comparison; any argmax
disagreement must sit on a logit gap below the logits tolerance.
"""
import os
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-4


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# Execution modes: the persistent step with its default attention (one item
# per query head while the context is short), the persistent step with the
# chunked attention split at every position, and the multi-kernel step.
MODES = {"persistent": 0, "persistent_chunked": 0, "persistent_pairs": 0, "multi": 1}
# Engine settings per mode: the chunked attention at every position; every
# input staged two elements per load (by default only inputs >= 4096 wide,
# which the tiny models do not have).
MODE_ENV = {"persistent_chunked": {"KL_ATTN_SHORT_MAX": "0"},
            "persistent_pairs": {"KL_STAGE_PAIR_MIN": "2"}}


def new_engine(K, img, cfg, mode=None):
    """An engine in execution mode `mode` (a MODES key; None: default)."""
    env = MODE_ENV.get(mode, {})
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        eng = K.Engine(img, cfg)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    if mode is not None:
        eng.set_mode(MODES[mode])
        assert eng.mode == MODES[mode]
    return eng


def teacher_forced(K, O, cfg, img, prompt, n_new, graph=True, mode=None):
    eng = new_engine(K, img, cfg, mode)
    eng.set_graph(graph)
    om = O.Model(img, cfg.family, cfg.quant)
    seq = [int(t) for t in prompt]
    worst, mismatches = 0.0, []
    for pos in range(len(prompt) + n_new - 1):
        nxt, lg = eng.step(seq[pos], pos)
        ref = om.step(seq[pos], pos)
        r = rel(lg, ref)
        worst = max(worst, r)
        assert r < LOGIT_RTOL, (cfg.name, pos, r)
        assert nxt == int(np.argmax(lg))  # the device argmax picks the first max
        if pos >= len(prompt) - 1:
            want = O.argmax(ref)
            if nxt != want:
                gap = abs(float(ref[nxt]) - float(ref[want]))
                mismatches.append((pos, gap))
                assert gap <= LOGIT_RTOL * np.max(np.abs(ref)), (cfg.name, pos, gap)
            seq.append(want)
    return eng, om, worst, mismatches


TINY_NAMES = ["tiny_llama2", "tiny_llama3", "tiny_q8", "tiny_qwen2", "tiny_qwen2_q8", "tiny_qwen3"]


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("name", TINY_NAMES)
def test_tiny_models_step_parity(K, O, gpu, name, mode):
    cfg = K.TINY[name]
    say("case", name, mode)
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    eng, om, worst, mm = teacher_forced(K, O, cfg, img, prompt, cfg.decode_steps, mode=mode)
    say(name, "worst logits rel err", worst, "argmax near-ties", mm)
    assert not mm
    # KV cache contents (K rotated) after the run
    for layer, pos in ((0, 0), (cfg.layers - 1, 3), (cfg.layers - 1, cfg.prompt_len)):
        for v in (False, True):
            a, b = eng.kv_row(layer, pos, v), om.kv_row(layer, pos, v)
            assert rel(a, b) < 1e-4


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("name", TINY_NAMES)
def test_tiny_models_generate_matches_oracle(K, O, gpu, name, mode):
    cfg = K.TINY[name]
    say("case", name, mode)
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, cfg.decode_steps)
    eng = new_engine(K, img, cfg, mode)
    got, ms = eng.generate(prompt, cfg.decode_steps)
    assert list(got) == list(want)
    # a second run on the same engine (state fully device-driven) repeats it
    got2, _ = eng.generate(prompt, cfg.decode_steps)
    assert list(got2) == list(want)


def test_graph_and_eager_agree_bitwise(K, O, gpu):
    cfg = K.TINY["tiny_qwen3"]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    a, b = K.Engine(img, cfg), K.Engine(img, cfg)
    a.set_mode(K.MODE_MULTI)
    b.set_mode(K.MODE_MULTI)
    b.set_graph(False)
    for pos, t in enumerate(list(prompt) + [5, 6, 7]):
        na, la = a.step(int(t), pos)
        nb, lb = b.step(int(t), pos)
        assert na == nb and np.array_equal(la, lb)


def test_persistent_is_deterministic_and_close_to_multi(K, O, gpu):
    """The persistent step sums each row in a fixed order: two engines (and two
    runs) agree bit for bit; the multi-kernel step differs only in rounding."""
    cfg = K.TINY["tiny_llama3"]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    a, b, m = K.Engine(img, cfg), K.Engine(img, cfg), K.Engine(img, cfg)
    a.set_mode(K.MODE_PERSISTENT)
    b.set_mode(K.MODE_PERSISTENT)
    wgs, threads, lds = a.launch_shape()
    say("persistent launch", wgs, threads, lds)
    assert wgs >= 1 and threads == 512 and lds > 0
    m.set_mode(K.MODE_MULTI)
    for pos, t in enumerate(list(prompt) + [11, 12, 13]):
        na, la = a.step(int(t), pos)
        nb, lb = b.step(int(t), pos)
        nm, lm = m.step(int(t), pos)
        assert na == nb and np.array_equal(la, lb)
        assert rel(la, lm) < LOGIT_RTOL
    ga, _ = a.generate(prompt, 16)
    gb, _ = a.generate(prompt, 16)
    assert list(ga) == list(gb)


def test_tag_epoch_wrap(K, O, gpu, monkeypatch):
    """The hand-off tags wrap after 2^24 launches (the wrapping launch clears
    the attention partials).  An engine whose epoch starts just before the
    wrap decodes across it, after split attention has begun (positions >= 64),
    bit for bit like one that starts at 0."""
    cfg = K.TINY["tiny_llama3"]  # 96 positions, 64-position attention chunks
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    monkeypatch.setenv("KL_ATTN_SHORT_MAX", "0")  # the chunked split at every position
    a = K.Engine(img, cfg)
    # engine creation runs 4 calibration steps; the wrap then falls near position 70
    monkeypatch.setenv("KL_EPOCH_START", str((1 << 24) - 4 - 70))
    b = K.Engine(img, cfg)
    monkeypatch.delenv("KL_EPOCH_START")
    for e in (a, b):
        e.set_mode(K.MODE_PERSISTENT)
    seq = [int(t) for t in prompt]
    for pos in range(cfg.seq_len - 1):
        t = seq[pos] if pos < len(seq) else seq[-1]
        na, la = a.step(t, pos)
        nb, lb = b.step(t, pos)
        assert na == nb and np.array_equal(la, lb), pos
        if pos + 1 >= len(seq):
            seq.append(int(na))


def test_l2_pull_changes_no_bits(K, O, gpu, monkeypatch):
    """Pulling W1/W3 rows into L2 during the attention phase only reads
    weights: an engine with the pull off decodes bit for bit like one with it
    on (cfg 2 shape, past the first 64-position chunk so some workgroups have
    no attention item)."""
    cfg = K.BASELINE["llama32_1b"]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg, 70)
    a = K.Engine(img, cfg)
    monkeypatch.setenv("KL_W13_TOUCH_ROWS", "0")
    b = K.Engine(img, cfg)
    monkeypatch.delenv("KL_W13_TOUCH_ROWS")
    for e in (a, b):
        e.set_mode(K.MODE_PERSISTENT)
    for pos, t in enumerate(list(prompt) + [3, 4, 5]):
        na, la = a.step(int(t), pos)
        nb, lb = b.step(int(t), pos)
        assert na == nb and np.array_equal(la, lb), pos
    ga, _ = a.generate(prompt, 8)
    gb, _ = b.generate(prompt, 8)
    assert list(ga) == list(gb)


@pytest.mark.parametrize("name", ["llama32_1b", "tiny_q8", "tiny_qwen2"])
def test_dynamic_classifier_rows_change_no_bits(K, O, gpu, monkeypatch, name):
    """The classifier's last rows handed out to workgroups at run time (the
    default from 2 MB of classifier per workgroup, as on Llama-3.2-1B: 20 % of
    the rows in blocks of 16), none of them (every row in the static split),
    or half of them in blocks of one row (every workgroup claims several):
    each row is computed the same way whichever workgroup takes it, so the
    logits agree bit for bit, step after step (the claim counter starts every
    launch at zero)."""
    cfg = K.ALL[name]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg, 6)
    engines = []
    for env in ({}, {"KL_CLS_DYN": "0"}, {"KL_CLS_DYN": "50", "KL_CLS_BLOCK": "1"}):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        engines.append(K.Engine(img, cfg))
        for k in env:
            monkeypatch.delenv(k)
    for e in engines:
        e.set_mode(K.MODE_PERSISTENT)
    for pos, t in enumerate(list(prompt) + [3, 4, 5, 6]):
        outs = [e.step(int(t), pos) for e in engines]
        for n, lg in outs[1:]:
            assert n == outs[0][0] and np.array_equal(lg, outs[0][1]), pos
    gens = [list(e.generate(prompt, 8)[0]) for e in engines]
    assert gens[1] == gens[0] and gens[2] == gens[0]
    om = O.Model(img, cfg.family, cfg.quant)
    assert gens[0] == [int(x) for x in om.generate(prompt, 8)]


def test_engine_rejects_bad_tokens(K, gpu):
    cfg = K.TINY["tiny_llama2"]
    eng = K.Engine(K.synth_image(cfg), cfg)
    with pytest.raises(K.KlError):
        eng.step(cfg.vocab, 0)
    with pytest.raises(K.KlError):
        eng.step(0, cfg.seq_len)
    with pytest.raises(K.KlError):
        eng.generate(np.array([1, cfg.vocab], np.int32), 2)


# ------------------------------------------- BASELINE shapes, full size -----
NORMS = 0.1  # full-size parity runs draw every norm weight from 1 + N(0, 0.1)


def test_cfg1_llama2_110m_full(K, O, gpu):
    """cfg 1 at full size: 16-token prompt + 128 greedy steps, teacher forced
    with non-unit norm weights, then 64 free-running greedy tokens on the
    benchmark's own model (norm weights 1.0)."""
    cfg = K.BASELINE["llama2_110m"]
    t = time.time()
    img = K.synth_image(cfg.with_(norm_std=NORMS))
    prompt = K.prompt_tokens(cfg)
    say("cfg1 image", img.nbytes, time.time() - t)
    eng, om, worst, mm = teacher_forced(K, O, cfg.with_(norm_std=NORMS), img, prompt,
                                        cfg.decode_steps)
    say("cfg1 worst logits rel err", worst, "near-ties", mm, "t", time.time() - t)
    assert not mm
    img = K.synth_image(cfg)
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, 64)
    for mode in MODES:
        eng = new_engine(K, img, cfg, mode)
        got, _ = eng.generate(prompt, 64)
        assert list(got) == list(want), mode


def first_flip(O, img, cfg, prompt, got, want):
    """Where two greedy sequences part: the position and the oracle's logit
    gap between the two tokens there (for the failure message)."""
    om = O.Model(img, cfg.family, cfg.quant)
    seq = [int(t) for t in prompt] + [int(t) for t in want]
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            pos = len(prompt) - 1 + i
            for p in range(pos):
                om.step(seq[p], p)
            ref = om.step(seq[pos], pos)
            return i, float(ref[b]) - float(ref[a])
    return None


def test_cfg2_llama32_1b_free_running_64(K, O, gpu):
    """The north-star bar on the benchmarked model itself (cfg 2, norm weights
    1.0 as generated for the bench): its 64-token prompt, then the first 64
    greedy tokens free-running, identical to the oracle's demo/main.cpp loop
    in both execution modes."""
    cfg = K.BASELINE["llama32_1b"]
    t = time.time()
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    assert len(prompt) == 64
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, 64)
    say("cfg2 oracle 64 tokens", time.time() - t)
    for name in MODES:
        eng = new_engine(K, img, cfg, name)
        got, ms = eng.generate(prompt, 64)
        say("cfg2", name, "tokens match:", list(got) == list(want), f"{ms:.1f} ms")
        if list(got) != list(want):
            pytest.fail(f"{name}: first flip (index, oracle gap) "
                        f"{first_flip(O, img, cfg, prompt, got, want)}")


def test_cfg2_llama32_1b_full(K, O, gpu):
    """cfg 2 at full size with non-unit norm weights: the 64-token prompt and
    64 greedy steps teacher forced, logits of every step within 1e-4, no
    argmax disagreement, in every mode."""
    cfg = K.BASELINE["llama32_1b"].with_(norm_std=NORMS)
    t = time.time()
    img = K.synth_image(cfg)
    say("cfg2 image", img.nbytes, time.time() - t)
    prompt = K.prompt_tokens(cfg)
    engs = {name: new_engine(K, img, cfg, name) for name in MODES}
    om = O.Model(img, cfg.family, cfg.quant)
    seq = [int(x) for x in prompt]
    worst = {n: 0.0 for n in engs}
    for pos in range(len(prompt) + 64 - 1):
        ref = om.step(seq[pos], pos)
        want = O.argmax(ref)
        for name, eng in engs.items():
            nxt, lg = eng.step(seq[pos], pos)
            r = rel(lg, ref)
            worst[name] = max(worst[name], r)
            assert r < LOGIT_RTOL, (name, pos, r)
            if pos >= len(prompt) - 1:
                assert nxt == want, (name, pos, float(ref[want]) - float(ref[nxt]))
        if pos >= len(prompt) - 1:
            seq.append(want)
    say("cfg2 worst logits rel err", worst, "t", time.time() - t)


@pytest.mark.parametrize("name,steps", [("llama2_7b_q8", 6), ("qwen25_15b", 6), ("qwen3_4b", 4)])
def test_other_baseline_shapes_full(K, O, gpu, name, steps):
    """cfg 3 / 4 / 5 at full size with non-unit norm weights, a few
    teacher-forced steps each, in both modes."""
    cfg = K.BASELINE[name].with_(norm_std=NORMS)
    t = time.time()
    img = K.synth_image(cfg)
    say(name, "image", img.nbytes, time.time() - t)
    prompt = K.prompt_tokens(cfg, 4)
    for mode in MODES:
        eng, om, worst, mm = teacher_forced(K, O, cfg, img, prompt, steps, mode=mode)
        say(name, "mode", mode, "worst logits rel err", worst, "near-ties", mm,
            "t", time.time() - t)
        assert not mm
        del eng, om


# ------------------------------------------------------- medium widths ----
# Shapes between the tiny models and the BASELINE configs, where a weight row
# spans several 4 KiB segments with a partial last one (fp32 D = 1536, F =
# 4608; int8 D = 5120, F = 5632: rows of 5 and 5.5 KiB), against the oracle.
MID = {
    "mid_llama3": lambda K: K.BASELINE["llama32_1b"].with_(
        name="mid_llama3", dim=2048, hidden_dim=4096, layers=2, heads=16, kv_heads=4,
        vocab=1000, seq_len=128, norm_std=NORMS, prompt_len=8, decode_steps=24),
    "mid_qwen2": lambda K: K.BASELINE["qwen25_15b"].with_(
        name="mid_qwen2", hidden_dim=4608, layers=2, vocab=1000, seq_len=128, norm_std=NORMS,
        prompt_len=8, decode_steps=24),
    "mid_q8": lambda K: K.BASELINE["llama2_7b_q8"].with_(
        name="mid_q8", dim=5120, hidden_dim=5632, layers=2, heads=40, kv_heads=40, vocab=1000,
        seq_len=64, norm_std=NORMS, prompt_len=6, decode_steps=12),
}


@pytest.mark.parametrize("name", list(MID))
def test_medium_width_parity(K, O, gpu, name):
    """Every step's logits within 1e-4 of the oracle and no argmax
    disagreement, teacher forced, in every mode; then free-running greedy
    tokens identical to the oracle's."""
    cfg = MID[name](K)
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg)
    for mode in MODES:
        say("case", name, mode)
        eng, om, worst, mm = teacher_forced(K, O, cfg, img, prompt, cfg.decode_steps, mode=mode)
        say(name, mode, "worst logits rel err", worst, "near-ties", mm)
        assert not mm
        for layer in (0, cfg.layers - 1):
            for pos in (0, cfg.prompt_len):
                for v in (False, True):
                    assert rel(eng.kv_row(layer, pos, v), om.kv_row(layer, pos, v)) < 1e-4
        del eng, om
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, cfg.decode_steps)
    got, _ = K.Engine(img, cfg).generate(prompt, cfg.decode_steps)
    assert list(got) == list(want)


# ----------------------------- long contexts on the benchmarked attention ----
def long_context(K, O, cfg, n_pos, check, n_greedy):
    """Teacher-forces `n_pos` seeded prompt positions through a persistent and
    a multi-kernel engine and the oracle in lockstep; logits compared at the
    positions in `check`, then `n_greedy` greedy steps compared at every step
    (no argmax disagreement allowed)."""
    img = K.synth_image(cfg)
    prompt = [int(t) for t in K.prompt_tokens(cfg, n_pos)]
    engs = {name: new_engine(K, img, cfg, name) for name in MODES}
    om = O.Model(img, cfg.family, cfg.quant)
    worst = {n: 0.0 for n in engs}
    seq = list(prompt)
    t = time.time()
    for pos in range(n_pos + n_greedy):
        ref = om.step(seq[pos], pos)
        look = pos in check or pos >= n_pos - 1
        for name, eng in engs.items():
            nxt, lg = eng.step(seq[pos], pos, want_logits=look)
            if look:
                r = rel(lg, ref)
                worst[name] = max(worst[name], r)
                assert r < LOGIT_RTOL, (cfg.name, name, pos, r)
                if pos >= n_pos - 1:
                    want = O.argmax(ref)
                    assert nxt == want, (name, pos, float(ref[want]) - float(ref[nxt]))
        if pos >= n_pos - 1:
            seq.append(O.argmax(ref))
        if pos % 500 == 0:
            say(cfg.name, "pos", pos, f"{time.time() - t:.1f} s")
    for name, eng in engs.items():
        for layer in (0, cfg.layers - 1):
            for p in (0, 513, n_pos - 1, n_pos + n_greedy - 1):
                for v in (False, True):
                    assert rel(eng.kv_row(layer, p, v), om.kv_row(layer, p, v)) < 1e-4
    say(cfg.name, "worst logits rel err", worst)


def test_long_context_qwen25_attention_shape(K, O, gpu):
    """cfg 4's attention (Qwen2: 12 Q / 2 KV heads of 128, QKV bias, 4096
    positions) at 2 layers with a narrow FFN and vocabulary: positions past
    512 and 1024 (9 and 17 chunks of 64 per kv head, where the persistent
    merge switches to several lanes and mergers per output, with a merger
    per 4 chunks up to 16 chunks and per 2 beyond) and a cache
    filled to 4000 positions followed by 8 greedy steps."""
    cfg = K.BASELINE["qwen25_15b"].with_(name="qwen25_attn_2l", layers=2, hidden_dim=512,
                                         vocab=1024, norm_std=NORMS)
    check = set(range(0, 4)) | set(range(188, 196)) | set(range(508, 520)) | set(range(700, 704)) \
        | set(range(1020, 1032)) | set(range(2040, 2052)) | set(range(3000, 3004))
    long_context(K, O, cfg, 4000, check, 8)


def test_long_context_llama32_attention_shape(K, O, gpu):
    """cfg 2's attention (32 Q / 8 KV heads of 64, rotate-half RoPE) at 2
    layers: past 512 and 1024 positions, to 1200."""
    cfg = K.BASELINE["llama32_1b"].with_(name="llama32_attn_2l", layers=2, hidden_dim=512,
                                         vocab=1024, seq_len=1216, norm_std=NORMS)
    check = set(range(0, 4)) | set(range(380, 390)) | set(range(508, 520)) | set(range(700, 704)) \
        | set(range(1020, 1032))
    long_context(K, O, cfg, 1190, check, 8)


def test_128_layer_image_runs_multi_kernel(K, O, gpu):
    """Hand-off tags hold the layer in 7 bits, so an image of 128 or more
    layers cannot run the persistent step: the engine must come up in the
    multi-kernel mode (refusing the persistent one) and match the oracle."""
    cfg = K.TINY["tiny_llama3"].with_(name="tiny_llama3_128l", layers=128, dim=64, hidden_dim=128,
                                      heads=2, kv_heads=1, vocab=300)
    img = K.synth_image(cfg)
    eng = K.Engine(img, cfg)
    assert eng.mode == K.MODE_MULTI
    with pytest.raises(K.KlError):
        eng.set_mode(K.MODE_PERSISTENT)
    om = O.Model(img, cfg.family, cfg.quant)
    for pos, t in enumerate(K.prompt_tokens(cfg, 6)):
        nxt, lg = eng.step(int(t), pos)
        assert rel(lg, om.step(int(t), pos)) < LOGIT_RTOL, pos
