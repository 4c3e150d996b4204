"""A Qwen3-architecture model served on the paged cache with the HIP kernels (PagedSession).

- fp32: logits equal the same model on eager attention with a contiguous DynamicCache (the
  reference session's cache) over a prefill and decode steps, batch of 3 (rtol/atol 1e-4).
- bf16: the kernels' attention against a float32 torch attention over a DynamicCache inside the
  same bf16 model (logits within 3e-2, identical greedy tokens).
- Scores of a round's action tokens, recovered from the LSE in one launch at the round's end
  (Algorithm 3), equal the eager attention probabilities of those tokens at their decode steps,
  max over each GQA group, averaged over the action tokens (rtol 1e-3).
- After end_round compresses, decoding continues with the logits of a DynamicCache compressed
  by index_select with the same kept positions (the reference's _compress, session.py:195-206).
Weights are random (no checkpoints); the architecture is transformers' Qwen3."""
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import AttentionInterface, DynamicCache, Qwen3Config, Qwen3ForCausalLM  # noqa: E402
from transformers.masking_utils import AttentionMaskInterface  # noqa: E402

from actkv.hf import PagedSession  # noqa: E402

pytestmark = pytest.mark.gpu


def _model(dtype, layers=3, hq=8, hkv=2, d=128, seed=0):
    cfg = Qwen3Config(vocab_size=211, hidden_size=256, intermediate_size=384, num_hidden_layers=layers,
                      num_attention_heads=hq, num_key_value_heads=hkv, head_dim=d, max_position_embeddings=4096)
    torch.manual_seed(seed)
    with torch.device("cuda"):
        m = Qwen3ForCausalLM(cfg)
    return m.to(dtype).eval()


def _fp32_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """Float32 reference attention over contiguous K/V (causal within the new tokens)."""
    q, k, v = query.float(), key.float(), value.float()
    g = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(g, 1).contiguous()
    v = v.repeat_interleave(g, 1).contiguous()
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scaling
    n, t = q.shape[2], k.shape[2]
    causal = torch.arange(t, device=q.device)[None, :] <= torch.arange(t - n, t, device=q.device)[:, None]
    s = s.masked_fill(~causal, float("-inf"))
    out = torch.matmul(torch.softmax(s, -1), v)
    return out.transpose(1, 2).to(query.dtype), None


AttentionInterface.register("fp32_ref", _fp32_attention)
AttentionMaskInterface.register("fp32_ref", lambda *a, **k: None)   # causality is in _fp32_attention


def _reference_run(model, impl, prompts, toks, keep=None, more=None):
    """Per sequence: prefill, decode toks; optionally compress to `keep` positions by
    index_select and decode `more` at logical positions.  Returns logits [1 + steps (+ more), V]."""
    model.set_attn_implementation(impl)
    outs = []
    with torch.no_grad():
        for b in range(prompts.shape[0]):
            cache = DynamicCache(config=model.config)
            lg = [model(input_ids=prompts[b:b + 1], past_key_values=cache, use_cache=True).logits[0, -1]]
            seen = prompts.shape[1]
            for t in toks[:, b]:
                lg.append(model(input_ids=t.view(1, 1), past_key_values=cache, use_cache=True,
                                position_ids=torch.tensor([[seen]], device="cuda")).logits[0, -1])
                seen += 1
            if keep is not None:
                idx = keep[b].to("cuda")
                for layer in cache.layers:
                    layer.keys = layer.keys.index_select(2, idx).contiguous()
                    layer.values = layer.values.index_select(2, idx).contiguous()
                for t in more[:, b]:
                    lg.append(model(input_ids=t.view(1, 1), past_key_values=cache, use_cache=True,
                                    position_ids=torch.tensor([[seen]], device="cuda")).logits[0, -1])
                    seen += 1
            outs.append(torch.stack(lg))
    return outs


def _tokens(B, n0, steps, seed, vocab=211):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(0, vocab, (B, n0), generator=g).cuda(),
            torch.randint(0, vocab, (steps, B), generator=g).cuda())


def test_fp32_logits_equal_eager_dynamic_cache():
    model = _model(torch.float32)
    B, n0, steps = 3, 45, 12
    prompts, toks = _tokens(B, n0, steps, seed=1)
    want = _reference_run(model, "eager", prompts, toks)
    sess = PagedSession(model, B, max_tokens=256, block_size=16)
    sess.kv.free = torch.randperm(sess.kv.num_blocks, generator=torch.Generator().manual_seed(3)).tolist()
    got = [sess.prefill(prompts)]
    for t in toks:
        got.append(sess.decode(t))
    got = torch.stack(got, 1)
    for b in range(B):
        torch.testing.assert_close(got[b], want[b], rtol=1e-4, atol=1e-4)
    assert all(sess.kv.seq_used[r] == n0 + steps for r in range(B))


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 128), (16, 2, 64), (4, 2, 256)])   # GQA 4 at head dim 128; GQA 8 at 64; the float32 path at 256
def test_bf16_logits_follow_fp32_attention(hq, hkv, d):
    model = _model(torch.bfloat16, hq=hq, hkv=hkv, d=d)
    B, n0, steps = 2, 300, 8
    prompts, toks = _tokens(B, n0, steps, seed=4)
    want = _reference_run(model, "fp32_ref", prompts, toks)
    sess = PagedSession(model, B, max_tokens=512)
    got = [sess.prefill(prompts)]
    for t in toks:
        got.append(sess.decode(t))
    got = torch.stack(got, 1).float()
    for b in range(B):
        w = want[b].float()
        tol = 3e-2 * max(1.0, w.abs().max().item())
        assert (got[b] - w).abs().max().item() < tol
        # the greedy token: the same as the reference's, or one whose reference logit is within the
        # tolerance of the reference's best (bf16 rounding of the attention output can flip a near-tie)
        pick = got[b].argmax(-1, keepdim=True)
        gap = w.max(-1).values - w.gather(-1, pick).squeeze(-1)
        assert bool((gap <= tol).all()), gap


def test_round_scores_equal_eager_attention_probabilities():
    model = _model(torch.float32, layers=2, hq=8, hkv=2)
    B, n0, steps = 2, 70, 9
    prompts, toks = _tokens(B, n0, steps, seed=5)
    in_action = [[j >= 3, j >= 5] for j in range(steps)]          # ragged action regions
    # reference: eager probabilities of each decode step, max over the GQA group
    model.set_attn_implementation("eager")
    want = torch.zeros(2, B, 2, n0 + steps, device="cuda")
    with torch.no_grad():
        for b in range(B):
            cache = DynamicCache(config=model.config)
            model(input_ids=prompts[b:b + 1], past_key_values=cache, use_cache=True)
            n_act = 0
            for j in range(steps):
                out = model(input_ids=toks[j, b].view(1, 1), past_key_values=cache, use_cache=True,
                            output_attentions=True)
                if in_action[j][b]:
                    n_act += 1
                    for layer, a in enumerate(out.attentions):
                        p = a[0, :, -1, :].float().view(2, 4, -1).amax(1)       # [Hkv, T]
                        want[layer, b, :, : p.shape[1]] += p
            want[:, b] /= n_act
    sess = PagedSession(model, B, max_tokens=256)
    sess.prefill(prompts, protected=True)
    sess.begin_round()
    for j in range(steps):
        sess.decode(toks[j], in_action=in_action[j])
    assert sess.n_action == [6, 4]
    sess._score_round()
    got = sess.lrfu.scores[:, :, :, : n0 + steps]
    torch.testing.assert_close(got, want, rtol=1e-3, atol=1e-6)
    assert sess.lrfu.n_seen.tolist() == [6, 4]


def test_decoding_after_compression_equals_index_select_cache():
    model = _model(torch.float32, layers=3)
    B, n0, steps, more_n = 2, 200, 24, 6
    prompts, toks = _tokens(B, n0, steps, seed=6)
    more = _tokens(B, 1, more_n, seed=7)[1]
    sess = PagedSession(model, B, max_tokens=512)
    sess.kv.free = torch.randperm(sess.kv.num_blocks, generator=torch.Generator().manual_seed(8)).tolist()
    got = [sess.prefill(prompts[:, :8], protected=True), sess.prefill(prompts[:, 8:])]
    sess.begin_round()
    for j in range(steps):
        got.append(sess.decode(toks[j], in_action=j >= steps - 10))
    free_before = len(sess.kv.free)
    perms = sess.end_round(budget=[60, 90])
    assert [len(p) for p in perms] == [8 + 60, 8 + 90]
    assert len(sess.kv.free) > free_before
    for p in perms:                                     # the protected prefix survives
        assert set(range(8)) <= set(p.tolist())
    for t in more:
        got.append(sess.decode(t))
    got = torch.stack(got[1:], 1)                       # from the full prompt on
    keep = [p.cpu() for p in perms]
    want = _reference_run(model, "eager", prompts, toks, keep=keep, more=more)
    for b in range(B):
        torch.testing.assert_close(got[b], want[b], rtol=1e-4, atol=1e-4)


def test_graph_decode_equals_eager_decode_across_a_compaction():
    """Decode steps replayed from a captured HIP graph give the eager session's logits and
    cache, step after step (the eager session's own launches run between the replays), also
    after a round's compaction rewrites the block tables."""
    model = _model(torch.bfloat16, layers=3)
    B, n0, steps = 3, 150, 14
    prompts, toks = _tokens(B, n0, steps, seed=9)
    order = torch.randperm(B * 40, generator=torch.Generator().manual_seed(10)).tolist()
    sessions = []
    for graph in (False, True):
        s = PagedSession(model, B, max_tokens=512, num_blocks=B * 40, graph=graph)
        s.kv.free = list(order)
        s.prefill(prompts[:, :4], protected=True)
        s.prefill(prompts[:, 4:])
        s.begin_round()
        sessions.append(s)
    eager, graph = sessions

    def step(t, act):
        le = eager.decode(t, in_action=act)
        lg = graph.decode(t, in_action=act)
        torch.testing.assert_close(lg.float(), le.float(), rtol=0, atol=2e-2)
        assert torch.equal(lg.argmax(-1), le.argmax(-1))

    for j in range(8):
        step(toks[j], j >= 5)
    assert graph._g is not None                     # replays after the first eager step
    for a, b in zip(eager._act, graph._act):        # the action tokens' q and lse
        torch.testing.assert_close(b[1], a[1], rtol=0, atol=1e-3)
    pe = eager.end_round(budget=[60, 70, 80])
    pg = graph.end_round(budget=[60, 70, 80])
    assert [p.tolist() for p in pe] == [p.tolist() for p in pg]
    eager.begin_round()
    graph.begin_round()
    for j in range(8, steps):
        step(toks[j], False)
    torch.cuda.synchronize()
    assert eager.kv.free == graph.kv.free and eager.kv.seq_used == graph.kv.seq_used
    assert {r: list(t) for r, t in eager.kv.tables.items()} == {r: list(t) for r, t in graph.kv.tables.items()}
    torch.testing.assert_close(graph.kv.kv.float(), eager.kv.kv.float(), rtol=0, atol=2e-2)
