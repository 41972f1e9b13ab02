"""BASELINE config 5 at its own shape: the random-init Qwen2-1.5B model
(28 layers, hidden 1536, 12 / 2 heads, FFN 8960, vocabulary 151936, RMSNorm
eps 1e-6, RoPE theta 1e4, bf16 weights ~ N(0, 0.02)) with 128 sequences of
2048-token paged contexts, the batch bench.py times.

* Logits of 4 of the sequences after their 2048-token prefill and after two
  teacher-forced decode steps of the whole 128-sequence batch, against
  transformers' Qwen2ForCausalLM (the model the reference's
  test/test_infer.py:17-34 compares with) run in fp32 from the same bf16
  weights: within 10 % of the reference logits' max magnitude, greedy tokens
  equal wherever the reference's top-2 margin exceeds twice the error. After
  the prefill the error must also stay below that of transformers' own bf16
  execution of the same weights.
  Why 10 % and not the 3 % of the 1-2 layer tests: the library keeps
  activations in bf16 between kernels, and over 28 layers and 2048-token
  contexts that rounding alone moves the logits by ~6 % of their max
  (measured; transformers in bf16 moves them by ~31 %). A wrong term, sign or
  index moves them by far more.
* Batch invariance: a decode step of 4 sequences alone gives the logits the
  same sequences got inside the 128-sequence decode step, to the same bf16
  tolerance. They are not bit-identical: the projections at M = 4 and M = 128
  run different GEMM kernels (other fp32 summation orders), and the flipped
  bf16 roundings grow over 28 layers to ~3 % of the logits' max (measured).
* 64 greedy steps in one llaisysQwen2ModelDecode call give the tokens of 64
  single llaisysQwen2ModelStep calls from an identical (forked) state.
* The same dimensions with 1 and 2 layers (hidden 1536, FFN 8960, vocabulary
  151936, 128 sequences x 2048 tokens, so the decode step runs the config-5
  kernels at M = 128): the logits of a prefill and two decode steps within
  3 % of the reference's max, per-layer error well under the 28-layer 10 %.
"""
import numpy as np
import pytest
import torch

import llaisys_amd as L
from llaisys_amd import DeviceType, MemcpyKind, RuntimeAPI, Tensor
from llaisys_amd.models import Qwen2, Qwen2Meta
from utils import to_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SHAPE = dict(nlayer=28, hs=1536, nh=12, nkvh=2, di=8960, voc=151936)
B, CTX, CHECKED = 128, 2048, 4
REL_TOL = 1e-1
DECODE_STEPS = 64


def _log(msg):
    print(f"[config5] {msg}", flush=True)


@pytest.fixture(scope="module")
def setup():
    maxseq = CTX + 8 + DECODE_STEPS + 16
    pages = (maxseq + 15) // 16
    meta = Qwen2Meta(**SHAPE, maxseq=maxseq, epsilon=1e-6, theta=10000.0, end_token=-1)
    _log("random-init model")
    model = Qwen2.random(meta, seed=5, std=0.02, num_blocks=2 * B * pages + CHECKED * pages + 64)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, SHAPE["voc"], CTX).tolist() for _ in range(B)]
    _log("prefill 128 x 2048")
    ids = [model.create_sequence()[0] for _ in range(B)]
    nxt, first_logits = [], None
    for s in range(0, B, 8):
        nxt += model.step(ids[s:s + 8], prompts[s:s + 8])
        if s == 0:
            first_logits = to_torch(model.logits())[:CHECKED].float().clone()
    return model, ids, prompts, nxt, first_logits


@pytest.fixture(scope="module")
def hf(setup):
    """transformers' Qwen2 in fp32 holding the library model's bf16 weights."""
    return hf_of(setup[0], SHAPE["nlayer"])


def hf_of(model, nlayer):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=SHAPE["voc"], hidden_size=SHAPE["hs"], intermediate_size=SHAPE["di"],
                      num_hidden_layers=nlayer, num_attention_heads=SHAPE["nh"],
                      num_key_value_heads=SHAPE["nkvh"], head_dim=128, max_position_embeddings=4096,
                      rms_norm_eps=1e-6, rope_theta=10000.0, tie_word_embeddings=False, attn_implementation="sdpa")
    _log("transformers model")
    with torch.device(DEV):
        ref = Qwen2ForCausalLM(cfg)
    api = RuntimeAPI(DeviceType.AMD)
    params = dict(ref.named_parameters())
    with torch.no_grad():
        for name in model.weight_names():
            t = Tensor(tensor=model.weight_handle(name))
            try:
                shape = t.shape()
                buf = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
                api.memcpy_sync(buf.data_ptr(), t.data_ptr(), buf.numel() * 2, MemcpyKind.D2D)
            finally:
                t._tensor = None  # borrowed handle: the model owns it
            params[name].copy_(buf.float())
    return ref.eval()


def hf_bf16_last_logits(ref, seqs):
    import copy

    half = copy.deepcopy(ref).to(torch.bfloat16)
    try:
        with torch.no_grad():
            return half(torch.tensor(seqs, device=DEV)).logits[:, -1].float()
    finally:
        del half
        torch.cuda.empty_cache()


def hf_last_logits(ref, seqs):
    with torch.no_grad():
        return ref(torch.tensor(seqs, device=DEV)).logits[:, -1].float()


def check(got, want):
    tol = REL_TOL * want.abs().max().item()
    err = (got - want).abs().max().item()
    assert err <= tol, f"max |logit diff| {err:.4g} > {tol:.4g}"


def check_tokens(toks, want, got):
    for t, row, mine in zip(toks, want, got):
        tol = (mine - row).abs().max().item()
        best = int(row.argmax())
        if t != best:
            assert (row[best] - row[t]).item() <= 2 * tol, f"token {t} vs reference {best}"


@pytest.mark.parametrize("nlayer", [1, 2])
def test_one_and_two_layers_at_config5_dims(nlayer):
    maxseq = CTX + 8
    pages = (maxseq + 15) // 16
    meta = Qwen2Meta(**{**SHAPE, "nlayer": nlayer}, maxseq=maxseq, epsilon=1e-6, theta=10000.0, end_token=-1)
    model = Qwen2.random(meta, seed=7 + nlayer, std=0.02, num_blocks=B * pages + 16)
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, SHAPE["voc"], CTX).tolist() for _ in range(B)]
    ids = [model.create_sequence()[0] for _ in range(B)]
    nxt = []
    for s in range(0, B, 16):
        nxt += model.step(ids[s:s + 16], prompts[s:s + 16])
    ref = hf_of(model, nlayer)
    hist = [list(p) for p in prompts[:CHECKED]]
    try:
        for step in range(2):  # decode steps of the whole batch (M = 128)
            feed = list(nxt)
            for i in range(CHECKED):
                hist[i].append(feed[i])
            nxt = model.step(ids, [[t] for t in feed])
            got = to_torch(model.logits())[:CHECKED].float()
            want = hf_last_logits(ref, hist)
            scale, err = want.abs().max().item(), (got - want).abs().max().item()
            _log(f"{nlayer} layer(s), decode step {step}: max|diff| {err:.3g} of max|logit| {scale:.3g}")
            assert err <= 3e-2 * scale
        assert L.device_error_flags() == 0
    finally:
        del ref
        del model
        torch.cuda.empty_cache()


def test_prefill_and_teacher_forced_decode_match_transformers(setup, hf):
    model, ids, prompts, nxt, first_logits = setup
    hist = [list(p) for p in prompts[:CHECKED]]
    want = hf_last_logits(hf, hist)
    bf16_err = (hf_bf16_last_logits(hf, hist) - want).abs().max().item()
    err = (first_logits - want).abs().max().item()
    _log(f"prefill logits: max|ref| {want.abs().max().item():.3g}, max|diff| {err:.3g}, "
         f"transformers bf16 max|diff| {bf16_err:.3g}")
    assert err <= bf16_err
    check(first_logits, want)
    check_tokens(nxt[:CHECKED], want, first_logits)
    feed = list(nxt)
    for step in range(2):
        # teacher-forced on the reference's choice for the checked sequences
        for i in range(CHECKED):
            feed[i] = int(want[i].argmax())
            hist[i].append(feed[i])
        nxt = model.step(ids, [[t] for t in feed])
        got = to_torch(model.logits())[:CHECKED].float()
        want = hf_last_logits(hf, hist)
        _log(f"decode step {step}: max|diff| {(got - want).abs().max().item():.3g}")
        check(got, want)
        check_tokens(nxt[:CHECKED], want, got)
        feed = list(nxt)
        setup[3][:] = nxt  # the batch's next tokens for the tests after this one


def test_decode_step_is_batch_invariant(setup):
    model, ids, prompts, nxt, _ = setup
    feed = list(nxt)
    hist = [model.length(i) for i in ids[:CHECKED]]
    # The same step in the 128 batch and for 4 forks alone (identical KV).
    forks = [model.fork(i) for i in ids[:CHECKED]]
    out_big = model.step(ids, [[t] for t in feed])
    big = to_torch(model.logits())[:CHECKED].float().clone()
    out_small = model.step(forks, [[t] for t in feed[:CHECKED]])
    small = to_torch(model.logits()).float()
    for f in forks:
        model.free(f)
    assert [model.length(i) for i in ids[:CHECKED]] == [h + 1 for h in hist]
    scale = big.abs().max().item()
    err = (big - small).abs().max().item()
    _log(f"batch 128 vs 4: max|diff| {err:.3g} of max|logit| {scale:.3g}")
    assert err <= REL_TOL * scale, f"{err} > {REL_TOL} x {scale}"
    for a, b_, row in zip(out_big[:CHECKED], out_small, big):
        if a != b_:
            assert abs(row[a].item() - row[b_].item()) <= 2 * err
    setup[3][:] = out_big


def test_multi_step_decode_equals_single_steps(setup):
    model, ids, _, nxt, _ = setup
    feed = list(nxt)
    forks = [model.fork(i) for i in ids]
    _log(f"{DECODE_STEPS} steps in one decode call")
    multi = model.decode(ids, feed, DECODE_STEPS)
    _log(f"{DECODE_STEPS} single steps")
    single = []
    cur = feed
    for _ in range(DECODE_STEPS):
        cur = model.step(forks, [[t] for t in cur])
        single.append(cur)
    single = np.asarray(single, np.int64)
    assert L.device_error_flags() == 0
    assert np.array_equal(multi, single), f"{int((multi != single).sum())} of {multi.size} tokens differ"
