"""The C-ABI from a plain C99 program (tests/c_abi/pkv_c_consumer.c, built by
__graft_entry__.build() or its Makefile): it includes only include/pkv.h and
the HIP runtime's C API, as an engine's FFI binding would (the reference's
Rust binds HIP through a C ABI, src/hip.rs:134-181). Host mode covers status
codes, the block allocator, the KV manager and argument checks; GPU mode
runs prompts admitted by the KV manager through append, gather (byte-exact),
the fused / unfused / no-allocation decode step (identical bytes), a
prefill over the same keys (decode row within 2e-3 + 1e-2 |want| of the
prefill's last row) and the same prefill with split keys (every row within
that tolerance of it)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "c_abi", "pkv_c_consumer")


def _run(mode):
    assert os.path.exists(EXE), "tests/c_abi/pkv_c_consumer is not built: run __graft_entry__.build()"
    r = subprocess.run([EXE, mode], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and r.stdout.rstrip().endswith("ok"), r.stdout + r.stderr


def test_c_consumer_host():
    if not os.path.exists(EXE):
        subprocess.run(["make", "-s", "-C", os.path.dirname(EXE)], check=True)
    _run("host")


@pytest.mark.gpu
def test_c_consumer_gpu():
    print("case C consumer gpu", flush=True)
    _run("gpu")
