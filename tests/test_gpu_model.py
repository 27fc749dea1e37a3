"""Model / engine end to end on the GPU: the kernels wired under the reference's
call surface, checked against the CPU oracle forward (fp32) and for the
chunked / prefix-cache / decode self-consistency the reference's own tests
assert (top-1 equal, top-20 overlap)."""
import sys

import pytest
import torch

from oracle import model as OM

pytestmark = pytest.mark.gpu

LAYERS, VOCAB = 2, 2048


@pytest.fixture(scope="module")
def model(pkg, gpu):
    # Untied lm_head: with a tied random embedding the residual stream keeps
    # the input token's own embedding, which then takes p ~ 1 and makes every
    # sampled log-probability ~0.  N(0, 0.1) gives logits of std ~3 over the
    # 2,048-token vocabulary: peaked but with entropy left to sample from.
    cfg = pkg.Qwen3Config(num_hidden_layers=LAYERS, vocab_size=VOCAB, tie_word_embeddings=False)
    torch.manual_seed(0)
    m = pkg.Qwen3ForCausalLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.uniform_(0.8, 1.2)
            elif "embed" in name:
                p.normal_(0, 0.25)
            elif "lm_head" in name:
                p.normal_(0, 0.1)
            elif p.dim() == 2:
                p.normal_(0, 0.02)
    m = m.to(gpu).to(torch.bfloat16).eval()
    m.allocate_global_kv_cache(num_blocks=64)
    return m


def _oracle_logits(model, ids):
    return OM.qwen3_logits(model.state_dict(), torch.as_tensor(ids)[None], LAYERS)[0]


def _prefill(pkg, model, seq, n):
    seq.num_scheduled_tokens = n
    ids, pos, cu_q, cu_k, mq, mk, bmap, bt = model._prepare_step([seq])
    with torch.no_grad():
        h = model.model.forward_prefill(ids, pos, cu_q, cu_k, mq, mk, bmap, bt)
        logits = model.lm_head(h).float()
    seq.kv_len += n
    seq.num_scheduled_tokens = 0
    return logits


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _topk_overlap(a, b, k=20):
    return len(set(torch.topk(a.float().cpu(), k).indices.tolist())
               & set(torch.topk(b.float().cpu(), k).indices.tolist()))


def test_prefill_logits_match_oracle(pkg, model):
    g = torch.Generator().manual_seed(1)
    toks = torch.randint(0, VOCAB, (300,), generator=g).tolist()
    bm = pkg.BlockManager(64)
    s = pkg.Sequence(toks)
    bm.allocate(s)
    print("[model] prefill vs oracle", flush=True)
    logits = _prefill(pkg, model, s, len(toks))
    ref = _oracle_logits(model, toks)
    assert _rel(logits, ref) < 3e-2
    assert (logits.argmax(-1).cpu() == ref.argmax(-1)).float().mean() > 0.9


def test_chunked_vs_unchunked_prefill(pkg, model):
    """The reference's chunked-prefill check: last-token logits of a ~500-token
    prompt prefilled whole vs in 256-token chunks: top-1 equal, top-20 >= 19."""
    g = torch.Generator().manual_seed(2)
    toks = torch.randint(0, VOCAB, (517,), generator=g).tolist()
    bm = pkg.BlockManager(64)
    a = pkg.Sequence(toks)
    bm.allocate(a)
    print("[model] chunked vs unchunked", flush=True)
    full = _prefill(pkg, model, a, len(toks))[-1]
    bm2 = pkg.BlockManager(64)
    b = pkg.Sequence(toks)
    bm2.allocate(b)
    while b.kv_len < len(toks):
        last = _prefill(pkg, model, b, min(256, len(toks) - b.kv_len))[-1]
        bm2.hash_blocks(b)
    assert last.argmax().item() == full.argmax().item()
    assert _topk_overlap(last, full) >= 19
    assert _rel(last, full) < 1e-2


def test_prefix_cached_prefill_matches_full_forward(pkg, model):
    """The reference's prefix-cache check: a prompt whose first 512 tokens hit
    the prefix cache, prefilled from kv_len=512, against the full forward."""
    g = torch.Generator().manual_seed(3)
    prefix = torch.randint(0, VOCAB, (512,), generator=g).tolist()
    bm = pkg.BlockManager(64)
    a = pkg.Sequence(prefix + [5, 6, 7])
    bm.allocate(a)
    _prefill(pkg, model, a, a.num_prompt_tokens)
    a.num_scheduled_tokens = a.num_prompt_tokens
    bm.hash_blocks(a)
    a.num_scheduled_tokens = 0
    toks = prefix + torch.randint(0, VOCAB, (40,), generator=g).tolist()
    b = pkg.Sequence(toks)
    bm.allocate(b)
    assert b.kv_len == 512 and b.block_table[:2] == a.block_table[:2]
    print("[model] prefix cached", flush=True)
    logits = _prefill(pkg, model, b, len(toks) - 512)
    ref = _oracle_logits(model, toks)[512:]
    assert logits[-1].argmax().item() == ref[-1].argmax().item()
    assert _topk_overlap(logits[-1], ref[-1]) >= 15
    assert _rel(logits, ref) < 3e-2


def test_teacher_forced_decode_matches_oracle_and_graph(pkg, model):
    g = torch.Generator().manual_seed(4)
    toks = torch.randint(0, VOCAB, (254,), generator=g).tolist()
    extra = torch.randint(0, VOCAB, (6,), generator=g).tolist()
    bm = pkg.BlockManager(64)
    s = pkg.Sequence(toks)
    bm.allocate(s)
    _prefill(pkg, model, s, len(toks))
    outs = []
    print("[model] teacher-forced decode", flush=True)
    for t in extra:                               # crosses the 256 page boundary
        s.append_token(t)
        bm.may_append(s)
        ids, pos, ctx, bt, slot = model._prepare_decode([s])
        with torch.no_grad():
            h = model.model.forward_decode(ids, pos, ctx, bt, slot)
            outs.append(model.lm_head(h)[0].float())
        s.kv_len += 1
    ref = _oracle_logits(model, toks + extra)[len(toks):]
    got = torch.stack(outs)
    assert _rel(got, ref) < 3e-2
    assert (got.argmax(-1).cpu() == ref.argmax(-1)).all()


def test_graph_decode_equals_eager(pkg, model):
    g = torch.Generator().manual_seed(5)
    bm = pkg.BlockManager(64)
    seqs = []
    for n in (100, 257, 31):
        s = pkg.Sequence(torch.randint(0, VOCAB, (n,), generator=g).tolist())
        bm.allocate(s)
        _prefill(pkg, model, s, n)
        s.append_token(7)
        bm.may_append(s)
        seqs.append(s)
    ids, pos, ctx, bt, slot = model._prepare_decode(seqs)
    print("[model] graph vs eager decode", flush=True)
    with torch.no_grad():
        eager = model.model.forward_decode(ids, pos, ctx, bt, slot).clone()
        model._init_cuda_graphs(max_bs=8, bt_width=4)
        model._capture_decode_graphs(batch_sizes=(4, 8))
        assert model._has_cuda_graphs
        first = None
        for _ in range(3):
            out = model._run_decode_graph(3, ids, pos, ctx, bt, slot).clone()
            torch.cuda.synchronize()
            first = out if first is None else first
            assert torch.equal(out, first)          # replays are deterministic
        # The graph runs the GEMMs at the padded batch (4 rows), eager at 3 rows:
        # hipBLASLt may pick different kernels, so compare within bf16 tolerance.
        assert (first.float() - eager.float()).abs().max().item() < 5e-2
    model._has_cuda_graphs = False
    model._graphs = {}


class _ReplaySpy:
    def __init__(self, graph):
        self.graph, self.calls = graph, 0

    def replay(self):
        self.calls += 1
        self.graph.replay()


def test_graph_decode_whole_units(pkg, model, monkeypatch):
    """Near-equal contexts replay the bucket's whole-unit graph (attention
    without merge launches), ragged ones the balanced graph; both match eager."""
    eng = sys.modules[type(model).__module__]
    monkeypatch.setattr(eng, "UNIT_GRAPH_MIN_BS", 4)
    g = torch.Generator().manual_seed(8)
    print("[model] whole-unit decode graphs", flush=True)
    with torch.no_grad():
        model._init_cuda_graphs(max_bs=8, bt_width=4)
        model._capture_decode_graphs(batch_sizes=(4, 8))
        assert model._has_cuda_graphs and set(model._graphs_units) == {4, 8}
        spy = _ReplaySpy(model._graphs_units[4])
        model._graphs_units[4] = spy
        for lens, units in (((300, 305, 310, 296), 1), ((40, 700, 300, 5), 0)):
            bm = pkg.BlockManager(64)
            seqs = []
            for n in lens:
                s = pkg.Sequence(torch.randint(0, VOCAB, (n,), generator=g).tolist())
                bm.allocate(s)
                _prefill(pkg, model, s, n)
                s.append_token(9)
                bm.may_append(s)
                seqs.append(s)
            ids, pos, ctx, bt, slot = model._prepare_decode(seqs)
            eager = model.model.forward_decode(ids, pos, ctx, bt, slot).clone()
            calls = spy.calls
            out = model._run_decode_graph_seqs(seqs).clone()
            torch.cuda.synchronize()
            assert spy.calls - calls == units
            assert (out.float() - eager.float()).abs().max().item() < 5e-2
            for s in seqs:
                bm.deallocate(s.block_table)
    model._has_cuda_graphs = False
    model._graphs = {}
    model._graphs_units = {}


def _oracle_logprobs(model, toks, plen, n_layers=LAYERS, mode="fp32"):
    """Oracle log-probabilities of the generated tokens toks[plen:], each
    scored at the previous position (temperature 1, no top-k: the sampling
    distribution of generate_continuous_with_logprobs, qwen3_naive.py:1636-1650)."""
    logits = OM.qwen3_logits(model.state_dict(), torch.as_tensor(toks[:-1])[None], n_layers,
                             mode=mode)[0]
    lp = torch.log_softmax(logits.double(), -1)
    tgt = torch.as_tensor(toks[plen:])
    return lp[plen - 1:].gather(-1, tgt[:, None])[:, 0]


# Log-probability bounds, 2x the measured deviation, against the oracle in the
# reference's bf16 numerics and against the exact fp32 oracle.  The deviation is
# set by the bf16 rounding of the logits (the reference's lm_head output is
# bf16 too): half an ulp is 1/32 nat at |x| in [8, 16), and a sampled token's
# logit and the top logits that dominate the log-sum-exp each carry one; the
# bf16 oracle rounds at the same points, but fp32 values that differ slightly
# upstream round to neighbouring bf16 values now and then (one full ulp).
LP_BF16_MAX, LP_BF16_MEAN = 0.12, 0.03
LP_FP32_MAX, LP_FP32_MEAN = 0.12, 0.035


def _assert_logprobs_match_oracle(model, toks, lps, plens, n_layers=LAYERS, rows=None, tag=""):
    """Engine log-probs against the oracle teacher-forced on the engine's own
    tokens, in both oracle modes."""
    d16, d32 = [], []
    for b in (range(len(toks)) if rows is None else rows):
        got = torch.tensor(lps[b], dtype=torch.float64)
        for mode, acc in (("bf16", d16), ("fp32", d32)):
            ref = _oracle_logprobs(model, toks[b], plens[b], n_layers, mode)
            assert got.shape == ref.shape
            acc.append((got - ref).abs())
    d16, d32 = torch.cat(d16), torch.cat(d32)
    print(f"[model] {tag} log-prob |engine - oracle| over {d16.numel()} tokens: "
          f"bf16 oracle max {d16.max().item():.5f} mean {d16.mean().item():.6f}; "
          f"fp32 oracle max {d32.max().item():.5f} mean {d32.mean().item():.6f}", flush=True)
    assert d16.max().item() <= LP_BF16_MAX and d16.mean().item() <= LP_BF16_MEAN
    assert d32.max().item() <= LP_FP32_MAX and d32.mean().item() <= LP_FP32_MEAN


def test_generate_continuous_and_logprobs(pkg, model):
    g = torch.Generator().manual_seed(6)
    prompts = [torch.randint(0, VOCAB, (1, n), generator=g) for n in (20, 300, 77)]
    print("[model] generate_continuous", flush=True)
    torch.manual_seed(0)
    seq_tokens, gen = model.generate_continuous(prompts, max_new_tokens=12, temperature=1.0,
                                                top_k=None)
    assert [len(x) for x in gen] == [12, 12, 12]
    assert model.last_stats["graph_steps"] > 0
    torch.manual_seed(0)
    toks, gen2, lps, plens = model.generate_continuous_with_logprobs(
        prompts, max_new_tokens=12, temperature=1.0, top_k=None)
    assert plens == [20, 300, 77] and [len(x) for x in lps] == [12, 12, 12]
    assert gen2 == gen                      # same seed, same tokens with or without log-probs
    _assert_logprobs_match_oracle(model, toks, lps, plens, tag="graphs+lookahead")


@pytest.mark.parametrize("mode", ["balanced_graph", "unit_graph", "eager", "lookahead"])
def test_engine_logprobs_match_oracle(pkg, model, monkeypatch, mode):
    """Every decode mode of the engine returns the log-probabilities the fp32
    oracle gives for the engine's own tokens: the balanced-schedule graphs
    (ragged contexts), the whole-unit graphs (near-equal contexts), eager
    decode, and the one-step lookahead."""
    eng = sys.modules[type(model).__module__]
    g = torch.Generator().manual_seed(21)
    if mode == "unit_graph":
        monkeypatch.setattr(eng, "UNIT_GRAPH_MIN_BS", 4)
        lens = (300, 305, 310, 296)
    else:
        lens = (20, 300, 77, 513)
    prompts = [torch.randint(0, VOCAB, (1, n), generator=g) for n in lens]
    model._has_cuda_graphs = False
    model.decode_lookahead = mode == "lookahead"
    try:
        torch.manual_seed(5)
        print(f"[model] engine vs oracle: {mode}", flush=True)
        toks, _, lps, plens = model.generate_continuous_with_logprobs(
            prompts, max_new_tokens=24, temperature=1.0, top_k=None, use_graphs=mode != "eager")
        st = model.last_stats
        if mode == "eager":
            assert st["graph_steps"] == 0
        else:
            assert st["graph_steps"] > 0
        if mode == "unit_graph":
            assert st["unit_graph_steps"] > 0
        if mode == "balanced_graph":
            assert st["unit_graph_steps"] == 0
        assert (st["lookahead_steps"] > 0) == (mode == "lookahead")
        _assert_logprobs_match_oracle(model, toks, lps, plens, tag=mode)
    finally:
        model.decode_lookahead = True
        model._has_cuda_graphs = False
        model._graphs, model._graphs_units = {}, {}


def test_generation_with_preemption(pkg, model):
    """A pool too small for every sequence at once forces LIFO preemption; all
    sequences still finish with the requested number of tokens."""
    model.allocate_global_kv_cache(num_blocks=6)
    try:
        g = torch.Generator().manual_seed(7)
        prompts = [torch.randint(0, VOCAB, (1, 250), generator=g) for _ in range(4)]
        print("[model] preemption", flush=True)
        _, gen = model.generate_continuous(prompts, max_new_tokens=20, temperature=1.0,
                                           top_k=20, use_graphs=False)
        assert [len(x) for x in gen] == [20] * 4
        assert model.last_stats["preemptions"] > 0
    finally:
        model._num_blocks = 0
        model.allocate_global_kv_cache(num_blocks=64)


@pytest.mark.parametrize("graphs,blocks", [(True, None), (False, None), (True, 6)])
def test_decode_lookahead_matches_synchronous_engine(pkg, model, graphs, blocks):
    """Launching decode step t+1 before step t's tokens are read back changes
    nothing: same tokens and log-probabilities as the synchronous engine, also
    with a pool small enough to force LIFO preemption."""
    g = torch.Generator().manual_seed(8)
    # Four ~250-token prompts + 40 tokens need 8 pages at the end: 6 forces preemption.
    prompts = [torch.randint(0, VOCAB, (1, n), generator=g) for n in (250, 240, 251, 245)]
    _lookahead_vs_sync(model, prompts, 40, graphs, blocks)


def _lookahead_vs_sync(model, prompts, new_tokens, graphs, blocks, oracle_rows=None):
    if blocks is not None:
        model.allocate_global_kv_cache(num_blocks=blocks)
    try:
        runs = []
        for la in (False, True):
            model.decode_lookahead = la
            torch.manual_seed(3)
            print(f"[model] lookahead={la} graphs={graphs} blocks={blocks}", flush=True)
            out = model.generate_continuous_with_logprobs(prompts, max_new_tokens=new_tokens,
                                                          temperature=1.0, top_k=None,
                                                          use_graphs=graphs)
            runs.append((out, dict(model.last_stats)))
        (t0, _, l0, p0), s0 = runs[0]
        (t1, _, l1, _), s1 = runs[1]
        assert t0 == t1 and l0 == l1
        assert all(t >= 0 for seq in t1 for t in seq)
        assert s1["lookahead_steps"] > 0 and s0["lookahead_steps"] == 0
        if blocks is not None:
            assert s1["preemptions"] > 0 and s1["preemptions"] == s0["preemptions"]
        if oracle_rows is not None:
            _assert_logprobs_match_oracle(model, t1, l1, p0, rows=oracle_rows,
                                          tag="lookahead after preemption")
    finally:
        model.decode_lookahead = True
        if blocks is not None:
            model._num_blocks = 0
            model.allocate_global_kv_cache(num_blocks=64)


@pytest.mark.parametrize("prompt_len", [1, 257])
def test_lookahead_readmitted_victim(pkg, model, prompt_len):
    """A victim preempted and re-admitted in the same scheduling round with a
    one-token prefill remainder (a one-token prompt, or a 257-token prompt
    whose first page is a prefix-cache hit) joins an all-decode step; the
    lookahead must feed it its last prompt token, not the token it sampled
    before it was rolled back.  Two sequences in a 5-page pool: at 512 tokens
    the second is its own LIFO victim, frees two pages and comes straight
    back."""
    g = torch.Generator().manual_seed(30 + prompt_len)
    prompts = [torch.randint(0, VOCAB, (1, prompt_len), generator=g) for _ in range(2)]
    new_tokens = 600 - prompt_len
    _lookahead_vs_sync(model, prompts, new_tokens, True, 5, oracle_rows=[1])
