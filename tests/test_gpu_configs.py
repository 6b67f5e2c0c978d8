"""Every BASELINE configuration through the product path (GPU).

Each config's golden greedy stream (tests/golden/<config>_p<P>_d<D>.json, written by
tests/golden/make_golden.py from the CPU oracle, the C++ restatement of Camelid's CPU
forward) is reproduced token for token by the path the benchmark times: the batched prefill
of the P-1 prompt tokens, then D steps of the device-side loop (camelid_hip_generate: one
replayed HIP graph per token, on-device embedding gather and argmax).  Mirrors the reference's
CPU<->GPU stream parity (tests/cuda_cpu_parity.rs:32-62) and full-forward parity at real dims
(src/cuda_resident/tests.rs:354).

Also here: the engine's documented switches (CAMELID_HIP_FUSED_GU, _FUSED_NORM, _GRAPHS,
_QKV_MERGED, _KQ_NORM_FUSED switched off; the opt-in _READ_AHEAD, _KV_AHEAD switched on;
_ATT_DG at each workgroup count) each against the same golden / oracle, and greedy ties
(duplicated lm_head rows) through the product argmax paths.
"""
import importlib.util
import json
from pathlib import Path

import numpy as np
import pytest

from camelid_amd.model import CONFIGS, ResidentSession, SyntheticModel, prompt_tokens, rope_tables, tiny_config

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _make_golden():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _golden(name):
    """The golden stream of `name` with the most decode steps."""
    files = list(GOLDEN.glob(f"{name}_p*_d*.json"))
    if not files:
        pytest.fail(f"no golden stream for {name}")
    return max((json.loads(f.read_text()) for f in files), key=lambda g: g["decode_len"])


_MODELS: dict = {}


def _model(name):
    """The config's synthetic model (generated once per test session; the big configs hold
    3.4-7.6 GB of weights)."""
    if name not in _MODELS:
        _MODELS.clear()
        _MODELS[name] = SyntheticModel.generate(CONFIGS[name])
    return _MODELS[name]


@pytest.mark.parametrize("name", ["tinyllama-1.1b", "llama-3.2-3b", "qwen3-8b", "mistral-7b-v0.3"])
def test_config_stream_matches_golden(name):
    """BASELINE configs[0], [2], [3], [4]: P-token prompt, D greedy tokens through the graph-
    replayed device loop, token-identical to the CPU oracle's stream.  The generator digest in
    the golden file pins the synthetic weights the stream was made from."""
    g = _golden(name)
    cfg = CONFIGS[name]
    model = _model(name)
    assert _make_golden().weights_digest(model) == g["weights_sha256_prefix"], "synthetic weights changed"
    prompt = prompt_tokens(cfg, g["prompt_len"])
    assert [int(t) for t in prompt] == g["prompt"]
    sess = ResidentSession(model, g["prompt_len"] + g["decode_len"], device_loop=True)
    try:
        toks = sess.generate(prompt, g["decode_len"])
    finally:
        sess.close()
    first_bad = next((i for i, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b), None)
    assert toks == g["tokens"], f"{name}: first differing step {first_bad} of {g['decode_len']}"


@pytest.mark.parametrize("switch,value", [("CAMELID_HIP_FUSED_GU", "0"), ("CAMELID_HIP_FUSED_NORM", "0"),
                                          ("CAMELID_HIP_READ_AHEAD", "1"), ("CAMELID_HIP_GRAPHS", "0"),
                                          ("CAMELID_HIP_KV_AHEAD", "1"), ("CAMELID_HIP_ATT_DG", "2"),
                                          ("CAMELID_HIP_ATT_O", "0"), ("CAMELID_HIP_ATT_SPLIT", "1")])
def test_switch_off_keeps_tinyllama_stream(monkeypatch, switch, value):
    """Each documented switch of the Q8_0 decode path set away from its default (the separate
    RMSNorm launch, the separate SwiGLU launch, the weight read-ahead workgroups, launches
    without a graph, the KV rows read by the qkv launch's idle waves, two attention workgroups
    per head of 64 dims instead of one, the output projection as its own launch instead of
    inside the attention launch, the one-launch split attention with the output projection at
    every position instead of from 1024 on): the TinyLlama golden stream (configs[0], 128 + 128)
    is still reproduced by the device loop."""
    monkeypatch.setenv(switch, value)
    test_config_stream_matches_golden("tinyllama-1.1b")


def test_split_attention_everywhere_keeps_llama3b_stream(monkeypatch):
    """configs[1] (Llama-3.2-3B-arch, heads of 128) with the one-launch split attention at every
    position (score slices of 128 positions below 1024 cache positions, the output projection's
    workgroups in the same launch): the golden stream is still reproduced."""
    monkeypatch.setenv("CAMELID_HIP_ATT_SPLIT", "1")
    test_config_stream_matches_golden("llama-3.2-3b")


@pytest.mark.parametrize("fused_split,att_o", [("0", "1"), ("1", "0")])
def test_split_attention_variants_keep_tinyllama_stream(monkeypatch, fused_split, att_o):
    """The split attention at every position in its other forms: two launches (scores, then
    outputs) with the output projection as its own launch, and one launch without the output
    projection's workgroups: the TinyLlama golden stream is still reproduced."""
    monkeypatch.setenv("CAMELID_HIP_ATT_SPLIT", "1")
    monkeypatch.setenv("CAMELID_HIP_ATT_FUSED_SPLIT", fused_split)
    monkeypatch.setenv("CAMELID_HIP_ATT_O", att_o)
    test_config_stream_matches_golden("tinyllama-1.1b")


def test_switch_off_qkv_merged_kquant_matches_oracle(monkeypatch):
    """At the C5 layer shape (hidden 4096, 32/8 heads of 128, ffn 12288, Q4_K_M), four K-quant
    decode layouts: the default (each RMSNorm inside the q|k+v and gate|up launches, whose other
    workgroups wait for it), CAMELID_HIP_KQ_NORM_FUSED=0 (a separate RMSNorm + Q8_K launch before
    the merged q|k+v launch and the gate|up launch), CAMELID_HIP_QKV_MERGED=0 (separate Q4_K
    q|k and Q6_K v launches, which also leaves the norm unfused) and the unfused layout with
    CAMELID_HIP_READ_AHEAD=1 (the norm launches' spare workgroups read the next weights ahead):
    per-layer hidden states, logits and tokens of each are bit-identical to the CPU oracle."""
    from oracle.oracle import OracleModel
    cfg = tiny_config(n_layers=2, hidden=4096, ffn_dim=12288, n_heads=32, n_kv_heads=8, head_dim=128, vocab=2048,
                      qk_norm=True, split_half=True, rope_theta=1e6, quant_scheme="q4_k_m", prompt_len=12)
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 32)
    orc.prefill(prompt[:-1])
    want = []
    tok, pos = int(prompt[-1]), len(prompt) - 1
    for _ in range(4):
        tok, hid, lg = orc.forward(tok, pos, hidden=True, logits=True)
        want.append((tok, hid, lg))
        pos += 1
    for merged, fused, ahead in (("1", "1", "0"), ("1", "0", "0"), ("0", "1", "0"), ("1", "0", "1")):
        monkeypatch.setenv("CAMELID_HIP_QKV_MERGED", merged)
        monkeypatch.setenv("CAMELID_HIP_KQ_NORM_FUSED", fused)
        monkeypatch.setenv("CAMELID_HIP_READ_AHEAD", ahead)
        sess = ResidentSession(model, 32)
        sess.engine.capture_hidden(True)
        sess.prefill(prompt[:-1])
        tok, pos = int(prompt[-1]), len(prompt) - 1
        for step, (t_o, hid_o, lg_o) in enumerate(want):
            tok = sess.step(tok, pos, logits=True)
            hid = sess.engine.read_hidden()
            assert np.array_equal(hid.view(np.uint32), hid_o.view(np.uint32)), (merged, fused, ahead, step)
            assert np.array_equal(sess.engine.last_logits.view(np.uint32), lg_o.view(np.uint32)), (
                merged, fused, ahead, step)
            assert tok == t_o
            pos += 1
        sess.close()


def test_split_attention_q4k_oproj_matches_oracle(monkeypatch):
    """At the C5 layer shape (hidden 4096 = 32 heads of 128, Q4_K_M: a Q4_K W_o), the decode
    attention split from the first position on, as one launch: with the Q4_K output
    projection's workgroups in that launch (they read the attention output as tagged f32 words
    and quantize it to Q8_K themselves) and, with CAMELID_HIP_ATT_O=0, as a launch of its own;
    per-layer hidden states, logits and tokens of both equal the CPU oracle's."""
    from oracle.oracle import OracleModel
    cfg = tiny_config(n_layers=2, hidden=4096, ffn_dim=12288, n_heads=32, n_kv_heads=8, head_dim=128, vocab=2048,
                      qk_norm=True, split_half=True, rope_theta=1e6, quant_scheme="q4_k_m", prompt_len=12)
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 32)
    orc.prefill(prompt[:-1])
    want = []
    tok, pos = int(prompt[-1]), len(prompt) - 1
    for _ in range(4):
        tok, hid, lg = orc.forward(tok, pos, hidden=True, logits=True)
        want.append((tok, hid, lg))
        pos += 1
    monkeypatch.setenv("CAMELID_HIP_ATT_SPLIT", "1")
    for att_o in ("1", "0"):
        monkeypatch.setenv("CAMELID_HIP_ATT_O", att_o)
        sess = ResidentSession(model, 32)
        sess.engine.capture_hidden(True)
        sess.prefill(prompt[:-1])
        tok, pos = int(prompt[-1]), len(prompt) - 1
        for step, (t_o, hid_o, lg_o) in enumerate(want):
            tok = sess.step(tok, pos, logits=True)
            hid = sess.engine.read_hidden()
            assert np.array_equal(hid.view(np.uint32), hid_o.view(np.uint32)), (att_o, step)
            assert np.array_equal(sess.engine.last_logits.view(np.uint32), lg_o.view(np.uint32)), (att_o, step)
            assert tok == t_o
            pos += 1
        sess.close()


def test_gate_up_group_loop_matches_oracle(monkeypatch):
    """At the C4 FFN shape (hidden 4096, ffn 14336: 448 gate/up row groups, more than the CUs
    hold 1024-thread workgroups at once), the norm-fused gate/up launch as one workgroup per CU,
    each taking its groups in turn (the next group's weights loaded during the current one's
    fold) and, with
    CAMELID_HIP_GU_LOOP=0, as 448 workgroups in two rounds; per-layer hidden states, logits and
    tokens of both equal the CPU oracle's, and so do the device loop's tokens."""
    from oracle.oracle import OracleModel
    cfg = tiny_config(n_layers=2, hidden=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128, vocab=2048,
                      rope_theta=1e6, prompt_len=12)
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 32)
    orc.prefill(prompt[:-1])
    want = []
    tok, pos = int(prompt[-1]), len(prompt) - 1
    for _ in range(4):
        tok, hid, lg = orc.forward(tok, pos, hidden=True, logits=True)
        want.append((tok, hid, lg))
        pos += 1
    for loop in ("1", "0"):
        monkeypatch.setenv("CAMELID_HIP_GU_LOOP", loop)
        sess = ResidentSession(model, 32)
        sess.engine.capture_hidden(True)
        sess.prefill(prompt[:-1])
        tok, pos = int(prompt[-1]), len(prompt) - 1
        for step, (t_o, hid_o, lg_o) in enumerate(want):
            tok = sess.step(tok, pos, logits=True)
            hid = sess.engine.read_hidden()
            assert np.array_equal(hid.view(np.uint32), hid_o.view(np.uint32)), (loop, step)
            assert np.array_equal(sess.engine.last_logits.view(np.uint32), lg_o.view(np.uint32)), (loop, step)
            assert tok == t_o
            pos += 1
        sess.close()
    # the device-side loop (graph replay) over the same steps
    monkeypatch.setenv("CAMELID_HIP_GU_LOOP", "1")
    sess = ResidentSession(model, 32, device_loop=True)
    assert sess.generate(prompt, len(want)) == [w[0] for w in want]
    sess.close()


def test_split_attention_q8_oproj_in_output_launch_matches_oracle(monkeypatch):
    """At the C4 layer shape (hidden 4096 = 32 heads of 128, 8 KV heads, Q8_0), the decode
    attention split from the first position on as two launches (scores, then output sums):
    with the Q8_0 output projection's workgroups in the output launch (2 rows per wave, reading
    the Q8_0 attention output as tagged words) and, with CAMELID_HIP_ATT_O=0, as a GEMV launch of
    its own; per-layer hidden states, logits and tokens of both equal the CPU oracle's."""
    from oracle.oracle import OracleModel
    cfg = tiny_config(n_layers=2, hidden=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=2048,
                      rope_theta=1e6, prompt_len=12)
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 32)
    orc.prefill(prompt[:-1])
    want = []
    tok, pos = int(prompt[-1]), len(prompt) - 1
    for _ in range(4):
        tok, hid, lg = orc.forward(tok, pos, hidden=True, logits=True)
        want.append((tok, hid, lg))
        pos += 1
    monkeypatch.setenv("CAMELID_HIP_ATT_SPLIT", "1")
    monkeypatch.setenv("CAMELID_HIP_ATT_FUSED_SPLIT", "0")
    for att_o in ("1", "0"):
        monkeypatch.setenv("CAMELID_HIP_ATT_O", att_o)
        sess = ResidentSession(model, 32)
        sess.engine.capture_hidden(True)
        sess.prefill(prompt[:-1])
        tok, pos = int(prompt[-1]), len(prompt) - 1
        for step, (t_o, hid_o, lg_o) in enumerate(want):
            tok = sess.step(tok, pos, logits=True)
            hid = sess.engine.read_hidden()
            assert np.array_equal(hid.view(np.uint32), hid_o.view(np.uint32)), (att_o, step)
            assert np.array_equal(sess.engine.last_logits.view(np.uint32), lg_o.view(np.uint32)), (att_o, step)
            assert tok == t_o
            pos += 1
        sess.close()


@pytest.mark.parametrize("dg",["1", "2", "4"])
def test_attention_workgroups_per_head_match_oracle(monkeypatch, dg):
    """CAMELID_HIP_ATT_DG: the decode attention with 1, 2 or 4 workgroups per query head (each
    recomputes the head's scores and denominator and sums 128 / DG output dims, staging only
    their V rows), head_dim 128, GQA 2:1, at positions 583..590 (the V ring's chunks hold 128,
    256 or 512 positions: several chunks plus a partial one and the 7-position tail): per-layer
    hidden states, logits and tokens bit-identical to the CPU oracle."""
    from oracle.oracle import OracleModel
    monkeypatch.setenv("CAMELID_HIP_ATT_DG", dg)
    cfg = tiny_config(n_layers=2, hidden=512, ffn_dim=1024, n_heads=4, n_kv_heads=2, head_dim=128, vocab=512,
                      prompt_len=584)
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 600)
    orc.prefill(prompt[:-1])
    sess = ResidentSession(model, 600)
    sess.engine.capture_hidden(True)
    sess.prefill(prompt[:-1])
    tok_o = tok_g = int(prompt[-1])
    pos = len(prompt) - 1
    for step in range(8):
        tok_o, hid_o, lg_o = orc.forward(tok_o, pos, hidden=True, logits=True)
        tok_g = sess.step(tok_g, pos, logits=True)
        assert np.array_equal(sess.engine.read_hidden().view(np.uint32), hid_o.view(np.uint32)), (dg, step)
        assert np.array_equal(sess.engine.last_logits.view(np.uint32), lg_o.view(np.uint32)), (dg, step)
        assert tok_g == tok_o
        pos += 1
    sess.close()


def _tied_max_model(cfg, period):
    """cfg's synthetic model with lm_head row r a copy of row r % period: every logit value
    occurs vocab/period times, so the greedy token is always a tie broken by the first index."""
    model = SyntheticModel.generate(cfg)
    rows = model.output.reshape(cfg.vocab, -1)
    model.output = np.ascontiguousarray(rows[np.arange(cfg.vocab) % period]).ravel()
    return model


@pytest.mark.parametrize("hidden,vocab,period", [(2048, 20000, 7), (256, 5000, 3)])
def test_greedy_ties_take_first_index(hidden, vocab, period):
    """greedy_sample's strict '>' (inference.rs:5912-5925): with the lm_head rows repeating every
    `period` rows, the maximum logit is reached by vocab/period rows spread over every lm_head
    workgroup; the product argmax (k_gemv_argmax partials + k_argmax_finish, two rows per wave
    at 20000 rows; the verify path's k_argmax_rows_part/finish) returns the first of them,
    which is the oracle's greedy token."""
    from oracle.oracle import OracleModel
    n_heads = hidden // 64
    cfg = tiny_config(hidden=hidden, ffn_dim=2 * hidden, n_heads=n_heads, n_kv_heads=max(1, n_heads // 4),
                      vocab=vocab, prompt_len=10)
    model = _tied_max_model(cfg, period)
    prompt = prompt_tokens(cfg)
    orc = OracleModel(model, 40)
    orc.prefill(prompt[:-1])
    sess = ResidentSession(model, 40)
    sess.prefill(prompt[:-1])
    tok_o = tok_g = int(prompt[-1])
    pos = len(prompt) - 1
    inputs, stream = [], []
    for _ in range(6):
        inputs.append(tok_g)
        tok_o, _, lg = orc.forward(tok_o, pos, logits=True)
        assert np.count_nonzero(lg == lg.max()) == len(range(int(np.argmax(lg)), vocab, period)) > 1
        tok_g = sess.step(tok_g, pos)
        assert tok_g == tok_o == int(np.argmax(lg)) < period
        stream.append(tok_g)
        pos += 1
    # the device loop and the verify path on the same inputs
    dev = ResidentSession(model, 40, device_loop=True)
    assert dev.generate(prompt, 6) == stream
    dev.close()
    base = len(prompt) - 1
    sess.engine.set_filled(base)
    cos, sin = rope_tables(cfg, base, 6)
    assert [int(t) for t in sess.engine.verify_batch(model.embed(inputs), cos, sin, base, cfg.scale())] == stream
    sess.close()
