"""The LAPrune decode path inside a (tiny, random) transformers Llama model.

* With ``mask_out = 0`` every candidate is selected, so the keep set is the
  whole cache and a LAPrune decode must equal the unpatched model's own
  full-sequence attention (same weights), step after step, across a 64-token
  encode flush.  Tolerance: 3e-2 of the largest logit (bf16 model; the two
  attention kernels round differently; measured 0.009).  Control: keeping
  only top-1 + sink + local moves the logits by far more (measured 0.94), so
  the comparison does see the attention.
  The same holds with G = 1, 2, 7 and 8 query heads per KV head (the kernel
  chain's per-head table, GQA scorer and top-k).
* A ragged batch decodes each sequence as that sequence alone (same
  tolerance: batched GEMMs may round differently from batch-1 GEMMs).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB = 1000


def _tiny(heads=8, kv_heads=2):
    from transformers import LlamaConfig
    hidden = 512 if 512 % heads == 0 else 64 * heads  # transformers wants heads | hidden
    return LlamaConfig(vocab_size=VOCAB, hidden_size=hidden, intermediate_size=1024,
                       num_hidden_layers=3, num_attention_heads=heads, num_key_value_heads=kv_heads,
                       head_dim=64, max_position_embeddings=4096, rope_theta=10000.0,
                       attn_implementation="sdpa")


def _codebooks(layers, seed=5):
    g = torch.Generator().manual_seed(seed)
    return {i: torch.randn(32, 256, 64, generator=g) * 0.1 for i in layers}


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-6))


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (8, 1), (4, 4), (8, 4), (7, 1)])  # G = 4, 8, 1, 2, 7
def test_keep_all_matches_dense_model(dev, heads, kv_heads):
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    print(f"tiny model: {heads} query heads, {kv_heads} KV heads", flush=True)
    cfg = _tiny(heads, kv_heads)
    ref = random_model(cfg, dev, seed=1)
    mod = random_model(cfg, dev, seed=1)
    for (n1, p1), (_, p2) in zip(ref.named_parameters(), mod.named_parameters()):
        assert torch.equal(p1, p2), n1
    s = LAPruneSettings(apply_layers=[1, 2],
                        retrieval=RetrievalConfig(mask_out=0.0, sink_size=4, local_window=64))
    lm = LAPruneLlama(mod, _codebooks([1, 2]), s, batch=1, capacity=512)
    g = torch.Generator().manual_seed(2)
    seq = torch.randint(0, VOCAB, (1, 300), generator=g).to(dev)
    P = 200
    lm.prefill(seq[:, :P - 1])
    ctl = LAPruneLlama(random_model(cfg, dev, seed=1), _codebooks([1, 2]),
                       LAPruneSettings(apply_layers=[1, 2], retrieval=RetrievalConfig(topk=1)),
                       batch=1, capacity=512)
    ctl.prefill(seq[:, :P - 1])
    worst_ctl = 0.0
    with torch.no_grad():
        for t in range(P - 1, 290):  # crosses the flush at 263 (199 + 64)
            got = lm.decode(seq[:, t:t + 1])
            want = ref(input_ids=seq[:, :t + 1], use_cache=False, logits_to_keep=1).logits[:, -1]
            assert _rel(got, want) < 3e-2, t
            worst_ctl = max(worst_ctl, _rel(ctl.decode(seq[:, t:t + 1]), want))
    assert worst_ctl > 0.3  # pruning the keep set is visible in the logits
    st = lm.states[1].cache
    assert st.lengths == [290] and st.encoded_lens == [263]
    assert lm.states[0].cache.encoded_lens == [290]  # dense layer: nothing to encode


def test_ragged_batch_matches_each_sequence_alone(dev):
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    cfg = _tiny()
    s = LAPruneSettings(apply_layers=[1, 2],
                        retrieval=RetrievalConfig(topk=32, sink_size=4, local_window=64))
    cbs = _codebooks([1, 2])
    batched = LAPruneLlama(random_model(cfg, dev, seed=3), cbs, s, batch=3, capacity=512)
    alone = LAPruneLlama(random_model(cfg, dev, seed=3), cbs, s, batch=1, capacity=512)
    g = torch.Generator().manual_seed(4)
    lens = [150, 90, 200]
    seqs = [torch.randint(0, VOCAB, (1, n + 80), generator=g).to(dev) for n in lens]
    for b, n in enumerate(lens):
        batched.prefill_row(b, seqs[b][:, :n])
    assert batched.lengths == lens
    outs = []
    for i in range(80):
        tok = torch.cat([sq[:, n + i:n + i + 1] for sq, n in zip(seqs, lens)])
        outs.append(batched.decode(tok))
    for b, n in enumerate(lens):
        alone.reset()
        alone.prefill(seqs[b][:, :n])
        for i in range(80):
            want = alone.decode(seqs[b][:, n + i:n + i + 1])
            assert _rel(outs[i][b:b + 1], want) < 5e-2, (b, i)
    assert batched.lengths == [n + 80 for n in lens]


def test_generate_shapes(dev):
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    s = LAPruneSettings(apply_layers=[2], retrieval=RetrievalConfig(topk=16))
    lm = LAPruneLlama(random_model(_tiny(), dev, seed=6), _codebooks([2]), s, batch=2,
                      capacity=256)
    ids = torch.randint(0, VOCAB, (2, 100), generator=torch.Generator().manual_seed(7))
    out = lm.generate(ids, max_new_tokens=12)
    assert out.shape == (2, 112) and torch.equal(out[:, :100].cpu(), ids)
    assert lm.lengths == [111, 111]


@pytest.mark.parametrize("ragged,select", [(False, "group"), (True, "group"), (True, "head")])
def test_captured_decode_matches_eager(dev, ragged, select):
    """Decode steps replayed from one captured graph (device plans, device
    positions, per-sequence flush ranges) follow the eager steps, across
    each sequence's 64-token flush."""
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    cfg = _tiny()
    s = LAPruneSettings(apply_layers=[1, 2],
                        retrieval=RetrievalConfig(topk=32, sink_size=4, local_window=64,
                                                  select=select))
    cbs = _codebooks([1, 2])
    B = 3
    eager = LAPruneLlama(random_model(cfg, dev, seed=8), cbs, s, batch=B, capacity=512)
    graph = LAPruneLlama(random_model(cfg, dev, seed=8), cbs, s, batch=B, capacity=512)
    lens = [150, 90, 200] if ragged else [150] * B
    g = torch.Generator().manual_seed(9)
    seqs = [torch.randint(0, VOCAB, (1, n + 80), generator=g).to(dev) for n in lens]
    for lm in (eager, graph):
        if ragged:
            for b, n in enumerate(lens):
                lm.prefill_row(b, seqs[b][:, :n])
        else:
            lm.prefill(torch.cat([sq[:, :n] for sq, n in zip(seqs, lens)]))
    for i in range(80):
        tok = torch.cat([sq[:, n + i:n + i + 1] for sq, n in zip(seqs, lens)])
        want = eager.decode(tok)
        got = graph.decode_graph(tok)
        assert _rel(got, want) < 3e-2, i
        assert torch.equal(graph.next_tokens(), got.argmax(dim=-1, keepdim=True))
    for a, b in zip(eager.states, graph.states):
        assert a.cache.lengths == b.cache.lengths
        assert a.cache.encoded_lens == b.cache.encoded_lens
    assert graph.states[1].cache.encoded_lens == [n + 64 for n in lens]


def test_generate_with_captured_steps(dev):
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    s = LAPruneSettings(apply_layers=[1, 2], retrieval=RetrievalConfig(topk=16))
    lm = LAPruneLlama(random_model(_tiny(), dev, seed=6), _codebooks([1, 2]), s, batch=2,
                      capacity=256)
    ids = torch.randint(0, VOCAB, (2, 100), generator=torch.Generator().manual_seed(7))
    out = lm.generate(ids, max_new_tokens=70, graph=True)
    assert out.shape == (2, 170) and torch.equal(out[:, :100].cpu(), ids)
    assert lm.lengths == [169, 169] and lm.states[1].cache.encoded_lens == [163, 163]


def test_over_capacity_raises_without_appending(dev):
    """A step that would exceed the capacity the decoders were sized for
    raises before any layer runs, so every layer keeps the same length."""
    from laprune_amd.llama import LAPruneLlama, LAPruneSettings, random_model
    from laprune_amd.retrieval import RetrievalConfig
    s = LAPruneSettings(apply_layers=[1, 2], retrieval=RetrievalConfig(topk=16))
    lm = LAPruneLlama(random_model(_tiny(), dev, seed=6), _codebooks([1, 2]), s, batch=2,
                      capacity=128)
    ids = torch.randint(0, VOCAB, (2, 129), generator=torch.Generator().manual_seed(8))
    with pytest.raises(RuntimeError, match="capacity"):
        lm.prefill(ids)
    assert all(st.cache.lengths == [0, 0] for st in lm.states)
    lm.prefill(ids[:, :127])
    lm.decode(ids[:, 127:128])
    assert lm.lengths == [128, 128]
    for call in (lambda: lm.decode(ids[:, 128:129]), lambda: lm.decode_graph(ids[:, 128:129]),
                 lambda: lm.prefill_row(0, ids[:1, :4])):
        with pytest.raises(RuntimeError, match="capacity"):
            call()
        assert all(st.cache.lengths == [128, 128] for st in lm.states)
        assert all(st.cache.encoded_lens == lm.states[1].cache.encoded_lens
                   for st in lm.states[1:])
