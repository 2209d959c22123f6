"""Host-side guards of the Llama drivers (lnship/llama.py), without a GPU:
every decode and eval entry point refuses positions or KV views beyond the
n_ctx cells its caches and rope table hold, before anything is launched."""
import types

import pytest

from lnship import llama


def _model(n_ctx, past=0):
    m = types.SimpleNamespace(cfg=types.SimpleNamespace(n_ctx=n_ctx), past=[past], n_seq=1)
    return m


@pytest.mark.parametrize("cls", [llama.LlamaLNS16, llama.LlamaLNS32])
def test_context_limit_raises(cls):
    m = _model(8)
    cls._check_ctx(m, 0, 8)          # fits exactly
    cls._check_ctx(m, 7, 1, 8)
    with pytest.raises(ValueError, match="context full"):
        cls._check_ctx(m, 7, 2)
    with pytest.raises(ValueError, match="context full"):
        cls._check_ctx(m, 8, 1)
    with pytest.raises(ValueError, match="KV view"):
        cls._check_ctx(m, 0, 1, 16)
    with pytest.raises(ValueError, match="KV view"):
        cls._check_ctx(m, 0, 1, 0)


def test_decode_entry_points_check_before_launch():
    # a full context is refused by the decode entry points themselves (the
    # checks run before any buffer, stream or library call)
    m = types.SimpleNamespace(cfg=types.SimpleNamespace(n_ctx=4), past=[4], n_seq=1, torch=None)
    m._check_ctx = types.MethodType(llama.LlamaLNS16._check_ctx, m)
    m.n_past = 4
    with pytest.raises(ValueError, match="context full"):
        llama.LlamaLNS16.decode_graph(m, 0)
    with pytest.raises(ValueError, match="context full"):
        llama.LlamaLNS16.decode_graph_batch(m, None)
    with pytest.raises(ValueError, match="context full"):
        llama.LlamaLNS16.eval(m, [1])
    with pytest.raises(ValueError, match="context full"):
        llama.LlamaLNS32.decode_graph(m, 0)
    with pytest.raises(ValueError, match="context full"):
        llama.LlamaLNS32.eval(m, [1])
