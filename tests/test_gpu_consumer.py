"""A compiled C++ caller of the C ABI (tests/consumer/abi_consumer.cc,
built against include/u15h.h and libu15h.so by __graft_entry__.build()):
the grouped q|k|v call a layer step makes, u15h_linear, and the
layer stack bound by the reference's tensor names, each checked by the
program itself against the CPU oracle; then the whole layer through
u15h_stack_layer_full, checked bit for bit against the same public calls
made by the program."""
import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = pathlib.Path(__file__).resolve().parent / "consumer" / "abi_consumer"


def test_cxx_consumer_of_the_abi():
    assert BIN.exists(), f"{BIN} is not built (__graft_entry__.build())"
    print("running", BIN, flush=True)
    p = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=240)
    print(p.stdout[-4000:], p.stderr[-2000:])
    assert p.returncode == 0, p.stdout[-2000:]
    assert "PASS (0 failed)" in p.stdout
    assert p.stdout.count("ok  ") >= 17
