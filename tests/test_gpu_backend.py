"""HipBackend (ember::Backend, device "hip") end to end against the oracle, on a synthetic Qwen3-shaped model.

The model: config 1's Qwen3-0.6B attention shape (hidden 1024, 16 q / 8 kv heads, head_dim 128, QK-RMSNorm, RoPE
theta 1e6) with the 0.6B model's MLP (intermediate 3072), 4 layers and an 8192-token tied vocabulary; N(0, 0.02)
weights written with the safetensors package in three dtypes (F32 projections, BF16 gate/up, F16 the rest), so the
backend's load-time conversions are exercised. The oracle composes its own pieces (rmsnorm, linear, append and
attention, as oracle/ restates them from the reference's CPU backend) with the GPU path's f16 roundings (xn, qkv,
attention output and the MLP activation stored as f16; cuda_backend.cu:350-366).

The run mirrors the reference's model tests: one sequence, a 512-token prompt then 128 greedy decode steps
(tests/test_model.cpp:95-101), and the uneven 300 / 37 / 363 chunks at block offset 3 with 8 greedy decodes
(:124-157). Logits within 2e-2 of the oracle's (max |d| / max |oracle|; the reference allows 3e-2 between its CPU and
CUDA backends); decode inputs follow the oracle's greedy tokens, and the GPU's greedy token equals the oracle's
wherever the oracle's top-two margin exceeds the logit error.
"""
import numpy as np
import pytest
import torch

import oracle
from ember_amd.backend import BackendOptions, SampleRequest, SamplingParams, create_backend
from ember_amd.paged_kv import StepBatch
from synthetic_model import OracleModel, write_model

pytestmark = pytest.mark.gpu

H, I, L, V = 1024, 3072, 4, 8192
NH, NKV, D = 16, 8, 128
Q, KV = NH * D, NKV * D
PAGE = 16


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """Writes the model directory; returns (dir, the oracle's f16 / f32 copies of every weight)."""
    d = tmp_path_factory.mktemp("qwen3_synthetic")
    return d, write_model(d, layers=L, vocab=V)


def _batch(tokens, start, first_block, n_pages, logit_rows):
    T = len(tokens)
    return StepBatch(tokens=list(tokens), positions=list(range(start, start + T)), query_start=[0, T],
                     context_len=[start + T], block_tables=list(range(first_block, first_block + n_pages)),
                     max_blocks=n_pages), np.arange(start, start + T, dtype=np.int32)


def _rel(got, want):
    return float(np.abs(got - want).max() / np.abs(want).max())


def _greedy_run(be, om, chunks, n_decode, first_block, rng):
    """Runs the prompt chunks then greedy decodes on both; returns (worst logit error, decisive agreements)."""
    greedy = [SampleRequest(SamplingParams(temperature=0.0))]
    prompt = rng.integers(3, V, sum(chunks)).tolist()
    n_pages = (sum(chunks) + n_decode + PAGE - 1) // PAGE
    otab = np.arange(n_pages, dtype=np.int32)[None, :]
    worst, decisive, length = 0.0, 0, 0
    steps = [prompt[sum(chunks[:i]):sum(chunks[:i + 1])] for i in range(len(chunks))]
    nxt = None
    for i in range(len(steps) + n_decode):
        toks = steps[i] if i < len(steps) else [nxt]
        b, pos = _batch(toks, length, first_block, (length + len(toks) + PAGE - 1) // PAGE, [len(toks) - 1])
        b.logit_rows = [len(toks) - 1]
        be.forward(b)
        got = be.logits(0)
        want = om.forward(toks, pos, otab, [len(toks) - 1])[0]
        err = _rel(got, want)
        worst = max(worst, err)
        srt = np.sort(want)
        gpu_tok = be.sample(greedy)[0]
        if srt[-1] - srt[-2] > 2 * np.abs(got - want).max():  # the oracle's choice is decisive at this error
            assert gpu_tok == int(np.argmax(want)), f"step {i}: greedy {gpu_tok} vs oracle {int(np.argmax(want))}"
            decisive += 1
        assert gpu_tok == int(np.argmax(got)), "sample(temperature 0) is the argmax of the backend's own logits"
        nxt = int(np.argmax(want))  # both follow the oracle's greedy token
        length += len(toks)
    return worst, decisive


def test_prefill_512_then_128_greedy_decodes(model):
    d, w = model
    be = create_backend(str(d), BackendOptions(max_batch_tokens=1024, max_seqs=8, kv_cache_tokens=64 * PAGE))
    assert be.num_kv_blocks() == 64 and be.vocab_size == V
    worst, decisive = _greedy_run(be, OracleModel(w), [512], 128, 0, np.random.default_rng(5))
    assert worst < 2e-2, f"logits differ from the oracle by {worst:.2e}"
    assert decisive >= 100, f"only {decisive} of 129 greedy choices were decisive"
    be.close()


def test_uneven_chunks_at_block_offset_3(model):
    """tests/test_model.cpp:124-157: chunks of 300, 37 (ending mid-page) and 363 on blocks from 3 (the oracle's
    sequence on blocks from 0), then 8 greedy decodes."""
    d, w = model
    be = create_backend(str(d), BackendOptions(max_batch_tokens=512, max_seqs=8, kv_cache_tokens=64 * PAGE))
    worst, decisive = _greedy_run(be, OracleModel(w), [300, 37, 363], 8, 3, np.random.default_rng(6))
    assert worst < 2e-2, f"logits differ from the oracle by {worst:.2e}"
    assert decisive >= 6
    be.close()


def test_capture_hidden_and_token_probs(model):
    d, w = model
    be = create_backend(str(d), BackendOptions(max_batch_tokens=64, max_seqs=4, kv_cache_tokens=8 * PAGE))
    be.set_capture_hidden(True)
    toks = [5, 17, 300, 4000, 8191]
    b, pos = _batch(toks, 0, 0, 1, [4])
    b.logit_rows = [2, 4]
    be.forward(b)
    hid = be.captured_hidden().reshape(L + 1, H)
    np.testing.assert_array_equal(hid[0], w["embed"][toks[-1]].astype(np.float32))  # the embedding, exactly
    assert np.isfinite(hid).all() and not np.array_equal(hid[1], hid[0])
    reqs = [SampleRequest(SamplingParams(temperature=0.7, top_k=50), counter=9), SampleRequest(SamplingParams(0.0))]
    lg = [be.logits(0), be.logits(1)]
    toks_, probs_ = oracle.sampling_distribution(lg[0], 0.7, 1.0, 50, 0.0)
    got = be.token_probs(reqs, [0, 0, 0, 1], [int(toks_[0]), int(toks_[10]), int(np.argsort(lg[0])[0]),
                                              int(np.argmax(lg[1]))])
    np.testing.assert_allclose(got[:2], probs_[[0, 10]], rtol=1e-4)
    assert got[2] == 0.0 and got[3] == 1.0  # outside the top-50; greedy row's argmax
    be.close()


def test_errors_raise(model, tmp_path):
    from ember_amd import EmberError

    d, _ = model
    with pytest.raises(EmberError, match="config.json"):
        create_backend(str(tmp_path), BackendOptions(kv_cache_tokens=256))
    be = create_backend(str(d), BackendOptions(max_batch_tokens=16, max_seqs=2, kv_cache_tokens=4 * PAGE))
    b, _ = _batch([1, V + 5], 0, 0, 1, [1])
    b.logit_rows = [1]
    with pytest.raises(EmberError, match="outside the vocabulary"):
        be.forward(b)
    with pytest.raises(EmberError, match="requests for"):
        be.sample([SampleRequest(), SampleRequest()])
    be.close()


def _multi_batch(seqs, lens, firsts, width, logit_rows):
    """One step of several sequences: seqs[i] are sequence i's new tokens, lens[i] its length before the step, its
    pages firsts[i], firsts[i] + 1, ... (table rows `width` wide, padded with page 0, never read past the context)."""
    tokens, positions, qs, ctx, tables = [], [], [0], [], []
    for toks, n, f in zip(seqs, lens, firsts):
        tokens += list(toks)
        positions += list(range(n, n + len(toks)))
        qs.append(qs[-1] + len(toks))
        ctx.append(n + len(toks))
        tables += [f + p for p in range(width)]
    return StepBatch(tokens=tokens, positions=positions, query_start=qs, context_len=ctx, block_tables=tables,
                     max_blocks=width, logit_rows=list(logit_rows))


def test_decode_steps_replay_one_graph_and_equal_eager(model):
    """A pure decode step (one token per sequence, every token a logit row in order) replays one hipGraph of the whole
    model step, as the reference's forward does (cuda_backend.cu:145-149, :402-454): padded to the token bucket with
    spare-block rows. Its real rows' logits equal the eager step's bit for bit (graphs off, same model, same steps):
    five sequences (bucket 6, one padding row) for 12 steps, then four (bucket 4) for 4. A step whose logit rows are not
    every token in order runs eagerly, and so does every step with graphs off (the replay counter shows which). Each
    layout is captured once and its graph relaunched after: the first bucket runs for more steps than the planner's
    staging ring has buffers, so the kept graph reads step integers staged through every buffer."""
    from ember_amd import _lib

    d, _ = model
    opts = dict(max_batch_tokens=256, max_seqs=8, kv_cache_tokens=64 * PAGE)
    bg = create_backend(str(d), BackendOptions(**opts))  # graphs on: the reference's default
    be = create_backend(str(d), BackendOptions(cuda_graphs=False, **opts))
    replays = _lib.lib().ember_backend_graph_replays
    captures = _lib.lib().ember_backend_graph_captures
    captured0 = captures()
    rng = np.random.default_rng(11)
    lens = [40, 70, 17, 33, 5]
    width = 8  # pages per table row: room for every prompt plus the decodes
    firsts = [i * width for i in range(len(lens))]
    prompts = [rng.integers(3, V, n).tolist() for n in lens]
    rows = np.cumsum(lens) - 1
    b = _multi_batch(prompts, [0] * 5, firsts, width, rows)
    for x in (bg, be):
        x.forward(b)  # a prefill step: eager in both
    nxt = [int(np.argmax(be.logits(r))) for r in range(5)]
    assert nxt == [int(np.argmax(bg.logits(r))) for r in range(5)]
    cur = list(lens)
    graphs_run = 0
    for step in range(16):
        S = 5 if step < 12 else 4
        logit_rows = [0, 2] if step == 3 else list(range(S))
        b = _multi_batch([[t] for t in nxt[:S]], cur[:S], firsts[:S], width, logit_rows)
        before = replays()
        be.forward(b)
        assert replays() == before, "graphs off: the step ran eagerly"
        bg.forward(b)
        graph_step = step != 3
        assert replays() == before + (1 if graph_step else 0)
        graphs_run += graph_step
        assert captures() - captured0 == (1 if step < 12 else 2), f"step {step}: one capture per layout"
        for i in range(len(logit_rows)):
            np.testing.assert_array_equal(bg.logits(i), be.logits(i), err_msg=f"step {step} row {i}")
        got = {r: int(np.argmax(be.logits(i))) for i, r in enumerate(logit_rows)}
        nxt = [got.get(r, 7) for r in range(S)] + nxt[S:]
        cur = [c + 1 for c in cur[:S]] + cur[S:]
    assert graphs_run == 15
    bg.close()
    be.close()


def test_full_shape_28_layers_full_vocabulary(tmp_path_factory):
    """The model bench.py --backend times: 28 layers and the tied 151,936-token vocabulary (1.19 GB of f16 weights).
    Two sequences prefill 24- and 40-token prompts in one batch, then run 3 greedy decode steps together (pure decode
    steps of every token a logit row: the whole-step graph replays). Every logit row is within 2e-2 of the oracle's
    composition run on that sequence alone; both follow the oracle's greedy tokens."""
    from ember_amd import _lib

    d = tmp_path_factory.mktemp("qwen3_full_shape")
    layers, vocab = 28, 151936
    w = write_model(d, layers=layers, vocab=vocab)
    assert len(w["layers"]) == layers and w["embed"].shape == (vocab, H)
    width = 8  # pages per sequence: 40 + 3 tokens fit in 3
    be = create_backend(str(d), BackendOptions(max_batch_tokens=128, max_seqs=2, kv_cache_tokens=2 * width * PAGE))
    assert be.vocab_size == vocab
    rng = np.random.default_rng(17)
    lens = [24, 40]
    prompts = [rng.integers(3, vocab, n).tolist() for n in lens]
    oms = [OracleModel(w, num_blocks=width) for _ in lens]
    otab = np.arange(width, dtype=np.int32)[None, :]
    replays = _lib.lib().ember_backend_graph_replays
    worst, nxt, cur = 0.0, [], [0, 0]
    for step in range(4):
        seqs = prompts if step == 0 else [[t] for t in nxt]
        rows = np.cumsum([len(t) for t in seqs]) - 1
        b = _multi_batch(seqs, cur, [0, width], width, rows)
        before = replays()
        be.forward(b)
        assert replays() == before + (0 if step == 0 else 1), "pure decode steps replay the whole-step graph"
        nxt = []
        for i, toks in enumerate(seqs):
            want = oms[i].forward(toks, np.arange(cur[i], cur[i] + len(toks), dtype=np.int32), otab, [len(toks) - 1])[0]
            got = be.logits(i)
            err = _rel(got, want)
            assert err < 2e-2, f"step {step} sequence {i}: logits differ from the oracle by {err:.2e}"
            worst = max(worst, err)
            nxt.append(int(np.argmax(want)))
        cur = [c + len(t) for c, t in zip(cur, seqs)]
    print(f"28 layers, vocabulary {vocab}: worst logit error {worst:.2e}")
    be.close()

