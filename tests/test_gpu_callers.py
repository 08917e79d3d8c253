"""The C ABI driven from C++ the way the reference's Rust would drive a hayai-hip crate.

tests/callers/ffn_caller.cpp replays the streamed decode's FFN call sequences
(crates/hayai-core/src/stream_infer.rs:1665-1722,3752-3864): prefetch into pinned slots,
DMA of the FFN regions, weight_bind, then the bound-GEMV form (sync_gemv_from_scratch), the
async form (begin_gemv_from_scratch + PendingGemv::wait) and the fused begin/finish seam,
each checked against the oracle FFN; then the error contract.  Built by build()
(tests/callers/Makefile); one child process per case.
"""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "callers", "hh_ffn_caller")


@pytest.mark.parametrize("ggml_type,d_model,d_ff,layers", [(12, 4096, 14336, 3), (16, 2048, 5632, 3), (2, 576, 1536, 4)])
def test_cpp_caller_replays_reference_sequences(ggml_type, d_model, d_ff, layers):
    print(f"[case] C++ caller type={ggml_type} {d_model}x{d_ff} layers={layers}", flush=True)
    assert os.path.exists(BIN), "run build() first (tests/callers/Makefile)"
    r = subprocess.run([BIN, str(ggml_type), str(d_model), str(d_ff), str(layers)], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "[caller] all ok" in r.stdout
