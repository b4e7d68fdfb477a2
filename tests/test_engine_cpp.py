"""The C++ engine API (ane-infer_amd/engine: GpuContext, GpuGraph, Q8Tensor,
upload_model_weights, encode_full_token_gpu, the GGUF reader ...) through its own C++ test
program, tests/cpp/test_engine.cpp (built by __graft_entry__.build() /
`make -C tests/cpp`).  CPU: the host-logic tests; GPU: everything, including
a tiny hybrid model's decode steps against the oracle."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "_build", "test_engine")


def _run(*args, timeout=240):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} not built: run __graft_entry__.build() or make -C tests/cpp")
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(res.stdout, res.stderr, flush=True)
    return res


def test_engine_host_logic():
    """Q8Tensor checks, greedy sampling, and the GGUF reader (metadata,
    tensors, dequant known answers, malformed files, the tiny model's GGUF)."""
    res = _run("--cpu-only")
    assert res.returncode == 0
    assert "FAIL" not in res.stdout
    for name in ("test_gguf_metadata_and_tensors", "test_gguf_dequant_known_answers",
                 "test_gguf_rejects_malformed_files", "test_gguf_config_and_weights_of_the_tiny_model"):
        assert f"PASS {name}" in res.stdout


@pytest.mark.gpu
def test_engine_on_gpu():
    res = _run()
    assert res.returncode == 0, res.stdout[-2000:]
    for name in ("test_gpu_context_creation", "test_upload_weights", "test_graph_single_gemv",
                 "test_q8_gemv_parallel_graph_replays", "test_graph_gemv_then_silu_mul",
                 "test_encode_full_token_gpu_matches_oracle", "test_gguf_model_decodes_like_the_direct_upload"):
        assert f"PASS {name}" in res.stdout
