"""GPU parity of the ggml boundary: a graph run through libggml-lnship.so's
graph_compute equals the oracle bit for bit on every node, in each xlns16
summation mode and for LNSHIP32 (tests/ggml_graph_check.py; one process per
mode because the backend reads GGML_LNS16_SUM once, as the reference builds
one library per mode)."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CHECK = os.path.join(HERE, "ggml_graph_check.py")


def _run(args, env):
    print("ggml_graph_check", *args, flush=True)
    r = subprocess.run([sys.executable, "-u", CHECK] + args, env=env, capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr[-3000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32"])
def test_ggml_graph_lnship16(mode):
    _run(["--mode", mode], dict(os.environ, GGML_LNS16_SUM=mode))


@pytest.mark.gpu
def test_ggml_graph_lnship32():
    _run(["--w32"], dict(os.environ))


@pytest.mark.gpu
def test_ggml_graph_sum_policy():
    # LNS16_SUM_POLICY: mixed summation modes per node (cuda/lns-cuda-context.cpp:221-269)
    _run(["--mode", "monte", "--policy", "MUL_MAT:ffn*=lpvip,SOFT_MAX=sum32,kq-0=base,qkv-1=monte"],
         dict(os.environ, GGML_LNS16_SUM="monte"))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["sum32", "monte"])
def test_ggml_graph_device_buffers(mode):
    # GGML_LNS_HIP_BUFFERS=device: tensors in the backend's HBM buffer type,
    # read and written in place
    _run(["--mode", mode, "--device-buffers"], dict(os.environ, GGML_LNS16_SUM=mode))


@pytest.mark.gpu
def test_ggml_graph_lnship32_device_buffers():
    _run(["--w32", "--device-buffers"], dict(os.environ))


@pytest.mark.gpu
@pytest.mark.parametrize("args", [["--mode", "sum32"], ["--mode", "monte"], ["--mode", "base", "--device-buffers"],
                                  ["--w32"], ["--w32", "--device-buffers"]],
                         ids=["sum32", "monte", "base-device", "lns32", "lns32-device"])
def test_ggml_graph_fused_pairs(args):
    # RMS_NORM -> MUL by the norm weight and MUL_MAT -> ADD of the residual
    # whose intermediates feed only the next node run as one launch each; the
    # outputs and (monte) the LFSR state after the graph equal the oracle's
    mode = args[1] if args[0] == "--mode" else "sum32"
    _run(args + ["--fused"], dict(os.environ, GGML_LNS16_SUM=mode))


@pytest.mark.gpu
@pytest.mark.parametrize("w32", [False, True])
def test_ggml_graph_data_movement(w32):
    # SCALE, and the KV-cache writes (SET_ROWS, CPY into an F16 view) and row
    # gathers (GET_ROWS) of a graph whose tensors live in HBM
    _run(["--movement"] + (["--w32"] if w32 else []), dict(os.environ, GGML_LNS16_SUM="sum32"))
