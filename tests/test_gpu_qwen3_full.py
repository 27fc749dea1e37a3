"""Qwen3-0.6B at full size on the GPU (28 layers, vocabulary 151,936,
random-init bf16 weights drawn as transformers initialises Qwen3: N(0, 0.02)
for every matrix and the tied embedding, ones for the norms), checked against
the fp32 CPU oracle:

* the full decode step of the 64-sequence serving batch (contexts
  U{1024..4096}, shuffled page tables, random pool contents), eager and as a
  replayed HIP graph, against ``oracle.model.qwen3_decode_step`` on sampled
  sequences (logits, final hidden state and the K/V rows the step stores);
* the GRPO rollout at reduced length (32 prompts x group 8 = 256 sequences of
  128 random tokens, 16 new tokens, T = 1, no top-k): the returned old
  log-probabilities against the oracle forward teacher-forced on the
  engine's own tokens;
* the same rollout shape under LIFO preemption (a pool too small for every
  sequence), with the lookahead and synchronous engines agreeing;
* the benchmarked rollout at its real length (256 x (128 + 1,024) tokens in
  the ~40 GB pool, and in a 1,200-page pool that forces LIFO preemption):
  contexts up to 1,152 keys over 5 pages, page crossings at batch 256, the
  whole-unit graphs at long contexts, old log-probs of sampled sequences and
  of LIFO victims against the oracle.

Reference: qwen3_naive.py:642-683 / :795-802 (decode step), :1068-1145
(graphs), :1257-1341 (scheduling, preemption), :1474-1679 (rollout with
log-probs).
"""
import pytest
import torch

from oracle import model as OM
from oracle import workloads as W

pytestmark = pytest.mark.gpu

LAYERS, VOCAB = 28, 151936
CHECK_LAYERS = (0, 1, 13, 27)
# Full-length rollout bars (log-probs, nats): 2x the measured deviation
# (2,048 tokens of sequences 0 and 255: max 0.031, mean 0.0064; a LIFO
# victim's 1,024: max 0.037, mean 0.0067).
FULL_MAX, FULL_MEAN = 0.08, 1.5e-2


def init_qwen3_weights(model, std=0.02):
    """transformers' Qwen3 initialisation: N(0, std) matrices and embedding,
    unit norm weights."""
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            else:
                p.normal_(0.0, std)


@pytest.fixture(scope="module")
def qwen3(pkg, gpu):
    torch.manual_seed(0)
    cfg = pkg.Qwen3Config()
    with torch.device(gpu):
        m = pkg.Qwen3ForCausalLM(cfg)
    init_qwen3_weights(m)
    m = m.to(torch.bfloat16).eval()
    yield m
    _release(m)


def _release(m):
    m._graphs, m._graphs_units, m._has_cuda_graphs = {}, {}, False
    m._graph_bufs = m._graph_pool = None
    for layer in m.model.layers:
        layer.self_attn.k_cache = layer.self_attn.v_cache = None
    m._num_blocks = 0
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _sd_cpu(m):
    return {k: v.detach().float().cpu() for k, v in m.state_dict().items()}


def test_config3_full_decode_step(pkg, qwen3):
    """The whole 28-layer decode step at the serving shape: B = 64, contexts
    U{1024..4096}, shuffled page tables; eager and HIP-graph replay agree,
    and sampled sequences match the fp32 oracle decode step."""
    m = qwen3
    dev = next(m.parameters()).device
    print("[full] config 3: building 28-layer pools", flush=True)
    w = W.decode_batch(seed=0, device=dev, batch=64, layers=LAYERS)
    nb = w["num_blocks"]
    for i, layer in enumerate(m.model.layers):
        layer.self_attn.k_cache = w["k_cache"][i]
        layer.self_attn.v_cache = w["v_cache"][i]
    m._num_blocks = nb
    try:
        ctx = w["context_lens"]
        bt = w["block_tables"]
        g = torch.Generator().manual_seed(1)
        ids = torch.randint(0, VOCAB, (64,), generator=g).to(dev)
        pos = ctx.long()
        slots = (bt.long().gather(1, (pos // 256)[:, None])[:, 0] * 256 + pos % 256).to(torch.int32)
        rows = [0, 21, 42, 63]
        ctx_c, bt_c = ctx.cpu(), bt.cpu()
        # Cached rows 0..ctx-1 of the sampled sequences, per layer (the step
        # writes only row ctx, so these are unchanged by it).
        k_ctx, v_ctx = [], []
        for layer in range(LAYERS):
            kl, vl = [], []
            for b in rows:
                n = int(ctx_c[b])
                pages = bt_c[b, :(n + 255) // 256].long().to(dev)
                kl.append(w["k_cache"][layer][pages].reshape(-1, 8, 128)[:n].float().cpu())
                vl.append(w["v_cache"][layer][pages].reshape(-1, 8, 128)[:n].float().cpu())
            k_ctx.append(kl)
            v_ctx.append(vl)
        print("[full] config 3: eager step, layer by layer", flush=True)
        # The eager step through the layers' own forward_decode, recording the
        # input and output of a few layers for the per-layer oracle check.
        layer_io = {}
        with torch.no_grad():
            hcur, res = m.model.embed_tokens(ids), None
            # A layer hands the next its MLP output as split-K partial products
            # (K.RowParts); dense() is that projection's bf16 output.
            dense = lambda t: t.dense() if isinstance(t, pkg.kernels.RowParts) else t  # noqa: E731
            for li, layer in enumerate(m.model.layers):
                if li in CHECK_LAYERS:
                    d_in = None if res is None else dense(hcur)[rows].float().cpu()
                    r_in = (hcur if res is None else res)[rows].float().cpu()
                hcur, res = layer.forward_decode(hcur, pos, ctx, bt, slots, res)
                if li in CHECK_LAYERS:
                    layer_io[li] = (d_in, r_in, dense(hcur)[rows].float().cpu(),
                                    res[rows].float().cpu())
            h, _ = m.model.norm(hcur, res)
            h = h.clone()
            logits = m.lm_head(h).float()
            assert torch.equal(h, m.model.forward_decode(ids, pos, ctx, bt, slots))
        torch.cuda.synchronize()
        kv_rows = [(torch.stack([w["k_cache"][l].view(-1, 8, 128)[int(slots[b])] for l in range(LAYERS)]),
                    torch.stack([w["v_cache"][l].view(-1, 8, 128)[int(slots[b])] for l in range(LAYERS)]))
                   for b in rows]
        print("[full] config 3: graph replay", flush=True)
        with torch.no_grad():
            m._init_cuda_graphs(max_bs=64, bt_width=bt.shape[1])
            m._capture_decode_graphs(batch_sizes=(64,))
            assert m._has_cuda_graphs
            outs = []
            for _ in range(3):
                outs.append(m._run_decode_graph(64, ids, pos, ctx, bt, slots).clone())
                torch.cuda.synchronize()
        for o in outs[1:]:
            assert torch.equal(o, outs[0])             # replays are deterministic
        gdiff = (outs[0].float() - h.float()).abs().max().item()
        print(f"[full] config 3: graph vs eager max |diff| {gdiff:.3e} "
              f"(bit-identical: {torch.equal(outs[0], h)})", flush=True)
        assert gdiff <= 5e-2
        def rel(a, b):
            return ((a - b).norm() / b.norm()).item()
        sd = _sd_cpu(m)
        print("[full] config 3: oracle, layer by layer", flush=True)
        # Each checked layer, fed the engine's own input, against the oracle
        # layer in the reference's bf16 numerics: rounding-level agreement.
        for li, (d_in, r_in, d_out, r_out) in layer_io.items():
            d_ref, r_ref, k_ref, v_ref = OM.qwen3_decode_layer(
                sd, li, d_in, r_in, pos.cpu()[rows], k_ctx[li], v_ctx[li], mode="bf16")
            errs = dict(mlp_out=rel(d_out, d_ref), residual=rel(r_out, r_ref),
                        k=max(rel(kv_rows[j][0][li].float().cpu(), k_ref[j]) for j in range(len(rows))),
                        v=max(rel(kv_rows[j][1][li].float().cpu(), v_ref[j]) for j in range(len(rows))))
            print(f"[full] config 3: layer {li}: {errs}", flush=True)
            assert max(errs.values()) <= 1e-2, (li, errs)
        print("[full] config 3: oracle decode step", flush=True)
        ref = {mode: OM.qwen3_decode_step(sd, ids.cpu()[rows], pos.cpu()[rows], k_ctx, v_ctx,
                                          LAYERS, mode=mode) for mode in ("bf16", "fp32")}
        got = logits.cpu()[rows]
        hid = h.float().cpu()[rows]
        stats = {mode: dict(logits=rel(got, r[0]), hidden=rel(hid, r[3]),
                            logit_max=(got - r[0]).abs().max().item())
                 for mode, r in ref.items()}
        drift = rel(ref["bf16"][0], ref["fp32"][0])
        print(f"[full] config 3: engine vs oracle {stats}; bf16 oracle vs fp32 oracle logits rel "
              f"{drift:.3e}", flush=True)
        # End to end, 28 random layers amplify rounding-level differences: the
        # reference's own bf16 numerics (the bf16 oracle) land about as far
        # from the exact fp32 step as the engine does.  The engine must stay
        # within that drift; an indexing or formula error is O(1).
        assert stats["fp32"]["logits"] <= 1.5 * drift + 5e-3
        assert stats["bf16"]["logits"] <= 2 * drift + 5e-3
        assert stats["fp32"]["hidden"] <= 1.5 * drift + 5e-3
        for j, b in enumerate(rows):
            top = torch.topk(ref["fp32"][0][j], 5).indices.tolist()
            assert int(got[j].argmax()) in top
    finally:
        _release(m)
        del w
        torch.cuda.empty_cache()


def _rollout_prompts(n_prompts, group, prompt_len, seed):
    g = torch.Generator().manual_seed(seed)
    base = [torch.randint(0, VOCAB, (1, prompt_len), generator=g) for _ in range(n_prompts)]
    return [p for p in base for _ in range(group)]


def _oracle_check(m, toks, lps, plens, rows, tag, max_bar=6e-2, mean_bar=1.5e-2):
    """Returned log-probs against the oracle teacher-forced on the engine's
    tokens: close to the reference's bf16 numerics, and within the bf16
    drift of the exact fp32 values (log-probs are ~ -11.9 nats here)."""
    sd = _sd_cpu(m)
    d = {"bf16": [], "fp32": []}
    for b in rows:
        print(f"[full] {tag}: oracle on sequence {b} ({len(toks[b])} tokens)", flush=True)
        got = torch.tensor(lps[b], dtype=torch.float64)
        for mode in d:
            logits = OM.qwen3_logits(sd, torch.as_tensor(toks[b][:-1])[None], LAYERS, mode=mode)[0]
            lp = torch.log_softmax(logits.double(), -1)
            tgt = torch.as_tensor(toks[b][plens[b]:])
            ref = lp[plens[b] - 1:].gather(-1, tgt[:, None])[:, 0]
            assert got.shape == ref.shape
            d[mode].append((got - ref).abs())
    d = {k: torch.cat(v) for k, v in d.items()}
    print(f"[full] {tag}: log-prob |engine - oracle| over {d['bf16'].numel()} tokens: "
          + "; ".join(f"{k} max {v.max().item():.5f} mean {v.mean().item():.6f}"
                      for k, v in d.items()), flush=True)
    # 2x the measured deviation (16 new tokens: max 0.027, mean 0.0064 nats).
    assert d["bf16"].max().item() <= max_bar and d["bf16"].mean().item() <= mean_bar
    assert d["fp32"].max().item() <= max_bar and d["fp32"].mean().item() <= mean_bar


def test_config5_rollout_reduced_length(pkg, qwen3):
    """Config 5's rollout at 16 new tokens: 256 sequences, graphs and the
    whole-unit schedule at batch 256, lookahead; old log-probs of sampled
    sequences against the fp32 oracle (log-probs near -ln V, 11.93 nats)."""
    m = qwen3
    m.allocate_global_kv_cache(num_blocks=1362)
    try:
        prompts = _rollout_prompts(32, 8, 128, seed=0)
        torch.manual_seed(2)
        print("[full] config 5 reduced: 256 x (128 + 16)", flush=True)
        toks, gen, lps, plens = m.generate_continuous_with_logprobs(
            prompts, max_new_tokens=16, temperature=1.0, top_k=None)
        st = dict(m.last_stats)
        print(f"[full] config 5 reduced: stats {st}", flush=True)
        assert [len(x) for x in gen] == [16] * 256 and plens == [128] * 256
        assert st["graph_steps"] > 0 and st["lookahead_steps"] > 0 and st["preemptions"] == 0
        # Group members share a prompt but sample independently.
        assert len({tuple(x) for x in gen[:8]}) > 1
        _oracle_check(m, toks, lps, plens, [0, 9, 130, 255], "config 5 reduced")
    finally:
        _release(m)


def test_config5_rollout_with_preemption(pkg, qwen3):
    """64 sequences of 128 + 160 tokens need 128 pages; a 100-page pool forces
    LIFO preemption.  Every sequence still gets its 160 tokens, the lookahead
    and synchronous engines agree token for token, and the log-probs of the
    last-admitted sequences (the LIFO victims) match the oracle."""
    m = qwen3
    m.allocate_global_kv_cache(num_blocks=100)
    try:
        prompts = _rollout_prompts(8, 8, 128, seed=3)
        runs = []
        for la in (False, True):
            m.decode_lookahead = la
            torch.manual_seed(4)
            print(f"[full] preemption run, lookahead={la}", flush=True)
            out = m.generate_continuous_with_logprobs(prompts, max_new_tokens=160,
                                                      temperature=1.0, top_k=None)
            runs.append((out, dict(m.last_stats)))
            print(f"[full] stats {runs[-1][1]}", flush=True)
        (t0, g0, l0, p0), s0 = runs[0]
        (t1, g1, l1, p1), s1 = runs[1]
        assert [len(x) for x in g1] == [160] * 64
        assert s1["preemptions"] > 0 and s0["preemptions"] == s1["preemptions"]
        assert t0 == t1 and l0 == l1
        _oracle_check(m, t1, l1, p1, [0, 62, 63], "config 5 preemption")
    finally:
        m.decode_lookahead = True
        _release(m)


def test_config5_rollout_full_length(pkg, qwen3):
    """Config 5 as benchmarked: 256 sequences x 1,024 new tokens (T = 1, no
    top-k) in the 1,362-page (~40 GB) pool with graphs, whole-unit graphs and
    the lookahead.  Contexts reach 1,152 keys on 5 pages; the old log-probs of
    the first and last sequences (2,048 tokens) match the oracle teacher-forced
    on the engine's tokens."""
    m = qwen3
    m.allocate_global_kv_cache(num_blocks=1362)
    try:
        prompts = _rollout_prompts(32, 8, 128, seed=0)
        torch.manual_seed(2)
        print("[full] config 5 full length: 256 x (128 + 1024)", flush=True)
        toks, gen, lps, plens = m.generate_continuous_with_logprobs(
            prompts, max_new_tokens=1024, temperature=1.0, top_k=None)
        st = dict(m.last_stats)
        print(f"[full] config 5 full length: stats {st}", flush=True)
        assert [len(x) for x in gen] == [1024] * 256 and [len(x) for x in lps] == [1024] * 256
        assert st["graph_steps"] > 900 and st["lookahead_steps"] > 900
        assert st["unit_graph_steps"] > 0 and st["preemptions"] == 0 and st["blocks_in_use"] == 0
        assert all(t >= 0 for seq in toks for t in seq)
        _oracle_check(m, toks, lps, plens, [0, 255], "config 5 full length",
                      max_bar=FULL_MAX, mean_bar=FULL_MEAN)
    finally:
        _release(m)


def test_config5_rollout_full_length_forced_preemption(pkg, qwen3):
    """The benchmarked forced-preemption run: 256 x 1,024 new tokens in 1,200
    pages (256 x 5 pages would need 1,280).  LIFO preemption fires, the
    lookahead and synchronous engines return the same tokens and log-probs,
    and a LIFO victim's log-probs (re-prefilled after its rollback) match the
    oracle."""
    m = qwen3
    m.allocate_global_kv_cache(num_blocks=1200)
    try:
        prompts = _rollout_prompts(32, 8, 128, seed=5)
        runs = []
        for la in (True, False):
            m.decode_lookahead = la
            torch.manual_seed(6)
            print(f"[full] config 5 full length, 1200 pages, lookahead={la}", flush=True)
            out = m.generate_continuous_with_logprobs(prompts, max_new_tokens=1024,
                                                      temperature=1.0, top_k=None)
            st = dict(m.last_stats)
            runs.append((out, st))
            print(f"[full] stats { {k: v for k, v in st.items() if k != 'preempted_seqs'} } "
                  f"victims {st['preempted_seqs'][:8]}...", flush=True)
        (t1, g1, l1, p1), s1 = runs[0]
        (t0, g0, l0, p0), s0 = runs[1]
        assert [len(x) for x in g1] == [1024] * 256
        assert s1["preemptions"] > 0 and s0["preemptions"] == s1["preemptions"]
        assert s1["preempted_seqs"] == s0["preempted_seqs"]
        assert t0 == t1 and l0 == l1
        victim = s1["preempted_seqs"][-1]
        _oracle_check(m, t1, l1, p1, [victim], "config 5 preemption victim",
                      max_bar=FULL_MAX, mean_bar=FULL_MEAN)
    finally:
        m.decode_lookahead = True
        _release(m)
