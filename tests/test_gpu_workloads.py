"""The BASELINE model workloads at their full sizes on the GPU, checked through
properties that hold bit for bit at any size (the CPU oracle takes about 2 s
per SmolLM2-shape token, so it checks the same paths at short prompts in
test_gpu_configs.py and in bench.py's default line).

  C2  SmolLM2-135M shape, sum32: the 128-token prompt, then 128 greedy decode
      steps replayed from HIP graphs equal the same steps run eagerly.
  C3  8 independent sequences with 256-token prompts and 64 greedy decode
      steps: in lpvip and sum32 every batched step (one launch per op for all
      8 sequences) equals each sequence decoded on its own; in monte, where
      the LFSR draws run across the sequences in graph order, the batched
      graph replays equal the batched eager steps from the same state.
  C4  the LNS32 Llama-1B shape with all 16 layers: the 512-token prompt, then
      24 greedy decode steps from HIP graphs equal the same steps run eagerly.

Each check compares complete logit vectors, bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def bits(t):
    torch.cuda.synchronize()
    return np.ascontiguousarray(t.cpu().numpy(), np.float32).view(np.uint32).copy()


def same(got, want, what):
    bad = np.nonzero(got != want)[0] if got.ndim == 1 else np.nonzero((got != want).ravel())[0]
    assert bad.size == 0, f"{what}: {bad.size}/{got.size} values differ, first at {bad[0]}"


def prompt(n_vocab, n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, n_vocab, n)]


@pytest.fixture(scope="module")
def smollm():
    from lnship import llama
    cfg = llama.SMOLLM2_135M
    print("\n[workloads] SmolLM2-135M synthetic weights", flush=True)
    return cfg, llama.synthetic_weights(cfg, seed=1234, std=0.02)


def test_c2_full_decode_graph_equals_eager(smollm):
    from lnship import llama
    cfg, w = smollm
    m = llama.LlamaLNS16(cfg, w, mode=O.SUM32)
    p = prompt(cfg.n_vocab, 128, 2024)
    print("[C2] 128-token prompt, 128 graph-replayed decode steps", flush=True)
    first = bits(m.eval(p))
    tok = int(np.argmax(first.view(np.float32)))
    graph = []
    for _ in range(128):
        out = m.decode_graph(tok)
        graph.append(bits(out))
        tok = int(torch.argmax(out))
    print("[C2] the same steps eagerly", flush=True)
    m.restart()
    same(bits(m.eval(p)), first, "C2 prompt logits")
    tok = int(np.argmax(first.view(np.float32)))
    for i, want in enumerate(graph):
        out = m.eval([tok])
        same(bits(out), want, f"C2 decode step {i}")
        tok = int(torch.argmax(out))


def _prefill8(m, cfg):
    last = []
    for s in range(8):
        last.append(bits(m.eval(prompt(cfg.n_vocab, 256, 300 + s), seq=s)))
    return last


@pytest.mark.parametrize("mode", ["lpvip", "sum32"])
def test_c3_full_batched_equals_single(smollm, mode):
    from lnship import llama
    cfg, w = smollm
    md = O.MODES[mode]
    print(f"[C3] {mode}: 8 x 256-token prompts, 64 batched graph decode steps", flush=True)
    b = llama.LlamaLNS16(cfg, w, mode=md, n_seq=8)
    last = _prefill8(b, cfg)
    tok = torch.tensor([int(np.argmax(x.view(np.float32))) for x in last], dtype=torch.int32, device="cuda")
    batched = []
    for _ in range(64):
        out = b.decode_graph_batch(tok)
        batched.append(bits(out).reshape(8, -1))
        tok = torch.argmax(out, dim=1).to(torch.int32)
    del b
    one = llama.LlamaLNS16(cfg, w, mode=md)
    for s in range(8):
        print(f"[C3] {mode}: sequence {s} on its own", flush=True)
        one.restart()
        same(bits(one.eval(prompt(cfg.n_vocab, 256, 300 + s))), last[s], f"C3 {mode} seq {s} prompt")
        tok = int(np.argmax(last[s].view(np.float32)))
        for i in range(64):
            out = one.decode_graph(tok)
            same(bits(out), batched[i][s], f"C3 {mode} seq {s} step {i}")
            tok = int(torch.argmax(out))


def test_c3_full_monte_batched_graph_equals_eager(smollm):
    from lnship import llama
    cfg, w = smollm
    print("[C3] monte: 8 x 256-token prompts, 64 batched graph decode steps", flush=True)
    m = llama.LlamaLNS16(cfg, w, mode=O.MONTE, n_seq=8)
    last = _prefill8(m, cfg)
    start = [int(np.argmax(x.view(np.float32))) for x in last]
    tok = torch.tensor(start, dtype=torch.int32, device="cuda")
    graph = []
    for _ in range(64):
        out = m.decode_graph_batch(tok)
        graph.append(bits(out))
        tok = torch.argmax(out, dim=1).to(torch.int32)
    lfsr = m.lfsr
    print("[C3] monte: the same steps eagerly from the same LFSR state", flush=True)
    m.restart()
    for s in range(8):
        same(bits(m.eval(prompt(cfg.n_vocab, 256, 300 + s), seq=s)), last[s], f"C3 monte seq {s} prompt")
    toks = start
    for i, want in enumerate(graph):
        out = m.eval_batch(toks)
        same(bits(out), want, f"C3 monte batched step {i}")
        toks = [int(t) for t in torch.argmax(out, dim=1)]
    assert m.lfsr == lfsr


def test_c4_full_lns32_graph_equals_eager():
    from lnship import llama
    cfg = llama.LLAMA_1B
    print("\n[C4] Llama-1B shape, 16 layers, xlns32 weights", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    e, f, d = cfg.n_embd, cfg.n_ff, cfg.head_dim
    nq, nkv = cfg.n_head * d, cfg.n_head_kv * d
    r = lambda *shape: torch.randn(*shape, generator=g, device="cuda") * 0.02
    w = {"tok_embd": r(cfg.n_vocab, e), "out_norm": torch.ones(e, device="cuda"), "layers": []}
    for _ in range(cfg.n_layer):
        w["layers"].append({"attn_norm": torch.ones(e, device="cuda"), "wq": r(nq, e), "wk": r(nkv, e),
                            "wv": r(nkv, e), "wo": r(e, nq), "ffn_norm": torch.ones(e, device="cuda"),
                            "w_gate": r(f, e), "w_up": r(f, e), "w_down": r(e, f)})
    m = llama.LlamaLNS32(cfg, w)
    del w
    p = prompt(cfg.n_vocab, 512, 4040)
    print("[C4] 512-token prompt, 24 graph-replayed decode steps", flush=True)
    first = bits(m.eval(p))
    tok = int(np.argmax(first.view(np.float32)))
    graph = []
    for _ in range(24):
        out = m.decode_graph(tok)
        graph.append(bits(out))
        tok = int(torch.argmax(out))
    print("[C4] the same steps eagerly", flush=True)
    m.restart()
    same(bits(m.eval(p)), first, "C4 prompt logits")
    tok = int(np.argmax(first.view(np.float32)))
    for i, want in enumerate(graph):
        out = m.eval([tok])
        same(bits(out), want, f"C4 decode step {i}")
        tok = int(torch.argmax(out))
