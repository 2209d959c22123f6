"""GPU parity of the whole decoder: lnship.llama against the CPU oracle of the
same graph (tests/llama_oracle.py), bit-exact logits after prefill and after
each decode step, for every summation mode (BASELINE configs 2 and 3 at a
small size; the full SmolLM2 shape is exercised by bench.py)."""
import numpy as np
import pytest

import oracle_lib as O
from llama_oracle import LlamaOracle16, LlamaOracle32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def tiny(n_ctx=512):
    from lnship.llama import LlamaConfig
    return LlamaConfig(n_layer=2, n_embd=64, n_head=4, n_head_kv=2, head_dim=16, n_ff=96, n_vocab=300, n_ctx=n_ctx)


def same(got, want, what):
    g = np.ascontiguousarray(got, np.float32).view(np.uint32)
    w = np.ascontiguousarray(want, np.float32).view(np.uint32)
    bad = np.nonzero(g != w)[0]
    assert bad.size == 0, f"{what}: {bad.size}/{g.size} logits differ, first at {bad[0]}"


@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32"])
def test_prefill_and_decode(mode):
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=99, std=0.2)
    m = O.MODES[mode]
    rng = np.random.default_rng(5)
    prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, 9)]
    print(f"\n[llama] {mode} prefill 9", flush=True)
    gpu = llama.LlamaLNS16(cfg, w, mode=m)
    cpu = LlamaOracle16(cfg, w, m)
    same(gpu.eval(prompt).cpu().numpy(), cpu.eval(prompt), f"{mode} prefill")
    tok = int(rng.integers(0, cfg.n_vocab))
    for step in range(3):
        print(f"[llama] {mode} decode {step}", flush=True)
        same(gpu.eval([tok]).cpu().numpy(), cpu.eval([tok]), f"{mode} decode {step}")
        tok = (tok * 7 + 3) % cfg.n_vocab
    # graph steps, an eager step between them (Monte: the device LFSR state
    # must be refreshed from the host's after it), then graph steps again
    for step, kind in enumerate(("graph", "graph", "graph", "eager", "graph", "graph")):
        print(f"[llama] {mode} {kind} decode {step}", flush=True)
        out = gpu.decode_graph(tok) if kind == "graph" else gpu.eval([tok])
        same(out.cpu().numpy(), cpu.eval([tok]), f"{mode} {kind} decode {step}")
        tok = (tok * 5 + 1) % cfg.n_vocab
    assert O.monte_get() == gpu.lfsr or m != O.MONTE


def test_kv_view_grows_past_256():
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=7, std=0.2)
    prompt = [i % cfg.n_vocab for i in range(254)]
    print("\n[llama] sum32 prompt 254 then decode across n_kv 256 -> 512", flush=True)
    gpu = llama.LlamaLNS16(cfg, w, mode=O.SUM32)
    cpu = LlamaOracle16(cfg, w, O.SUM32)
    same(gpu.eval(prompt).cpu().numpy(), cpu.eval(prompt), "prefill 254")
    for step, tok in enumerate((3, 11, 17)):
        same(gpu.decode_graph(tok).cpu().numpy(), cpu.eval([tok]), f"decode {254 + step}")


@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32"])
def test_batched_sequences(mode):
    """BASELINE config 3 in small: independent sequences with their own KV
    caches, each prompt run on its own, then decode steps that take one token
    per sequence (attention batched over sequences)."""
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=31, std=0.2)
    m = O.MODES[mode]
    rng = np.random.default_rng(17)
    gpu = llama.LlamaLNS16(cfg, w, mode=m, n_seq=3)
    cpu = LlamaOracle16(cfg, w, m, n_seq=3)
    for s, n in enumerate((5, 9, 7)):
        prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, n)]
        print(f"\n[llama] {mode} seq {s} prefill {n}", flush=True)
        same(gpu.eval(prompt, seq=s).cpu().numpy(), cpu.eval(prompt, seq=s), f"{mode} seq {s} prefill")
    toks = [int(t) for t in rng.integers(0, cfg.n_vocab, 3)]
    for step in range(3):
        print(f"[llama] {mode} batched decode {step}", flush=True)
        same(gpu.eval_batch(toks).cpu().numpy(), cpu.eval_batch(toks), f"{mode} batched decode {step}")
        toks = [(t * 7 + 3 + i) % cfg.n_vocab for i, t in enumerate(toks)]
    for step in range(3):
        print(f"[llama] {mode} batched graph decode {step}", flush=True)
        dev = torch.tensor(toks, dtype=torch.int32, device="cuda")
        same(gpu.decode_graph_batch(dev).cpu().numpy(), cpu.eval_batch(toks), f"{mode} batched graph {step}")
        toks = [(t * 5 + 1 + i) % cfg.n_vocab for i, t in enumerate(toks)]
    assert gpu.past == cpu.past
    assert O.monte_get() == gpu.lfsr or m != O.MONTE


def test_lns32_prefill_and_decode():
    """BASELINE config 4 in small: the LNS32 decoder (F32 embedding rows,
    xlns32 ops, 4-byte weights, xlns32 KV cache of half-rounded values)."""
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=77, std=0.2)
    rng = np.random.default_rng(8)
    prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, 9)]
    print("\n[llama32] prefill 9", flush=True)
    gpu = llama.LlamaLNS32(cfg, w)
    cpu = LlamaOracle32(cfg, w)
    same(gpu.eval(prompt).cpu().numpy(), cpu.eval(prompt), "lns32 prefill")
    tok = int(rng.integers(0, cfg.n_vocab))
    for step in range(3):
        print(f"[llama32] decode {step}", flush=True)
        same(gpu.eval([tok]).cpu().numpy(), cpu.eval([tok]), f"lns32 decode {step}")
        tok = (tok * 7 + 3) % cfg.n_vocab
    for step in range(2):
        print(f"[llama32] graph decode {step}", flush=True)
        same(gpu.decode_graph(tok).cpu().numpy(), cpu.eval([tok]), f"lns32 graph decode {step}")
        tok = (tok * 5 + 1) % cfg.n_vocab


def test_lns32_graph_decode_across_kv_boundary():
    """LNS32 decode replayed from HIP graphs while the KV view grows from 256
    to 512 cells (a new graph is captured for the second view), after a
    prefill that already sized every buffer and the device scratch."""
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=13, std=0.2)
    prompt = [(i * 7) % cfg.n_vocab for i in range(253)]
    print("\n[llama32] prompt 253 then graph decode across n_kv 256 -> 512", flush=True)
    gpu = llama.LlamaLNS32(cfg, w)
    cpu = LlamaOracle32(cfg, w)
    same(gpu.eval(prompt).cpu().numpy(), cpu.eval(prompt), "lns32 prefill 253")
    for step, tok in enumerate((5, 9, 2, 40)):
        print(f"[llama32] graph decode at position {253 + step}", flush=True)
        same(gpu.decode_graph(tok).cpu().numpy(), cpu.eval([tok]), f"lns32 graph decode {253 + step}")
    assert sorted(gpu._graphs) == [256, 512]


def test_buffer_growth_drops_captured_graphs():
    """A prefill longer than any before grows the activation buffers; the
    graphs captured against the old buffers are dropped, and the next graph
    decode is captured anew and still equals the oracle."""
    from lnship import llama
    cfg = tiny()
    w = llama.synthetic_weights(cfg, seed=21, std=0.2)
    gpu = llama.LlamaLNS16(cfg, w, mode=O.SUM32)
    cpu = LlamaOracle16(cfg, w, O.SUM32)
    print("\n[llama] prefill 3, graph decode, prefill 40, graph decode", flush=True)
    same(gpu.eval([1, 2, 3]).cpu().numpy(), cpu.eval([1, 2, 3]), "prefill 3")
    same(gpu.decode_graph(4).cpu().numpy(), cpu.eval([4]), "graph decode 3")
    assert gpu._graphs
    long_prompt = [(i * 3) % cfg.n_vocab for i in range(40)]
    same(gpu.eval(long_prompt).cpu().numpy(), cpu.eval(long_prompt), "prefill 40")
    assert not gpu._graphs
    same(gpu.decode_graph(7).cpu().numpy(), cpu.eval([7]), "graph decode 44")
