"""Runs the C++ host-interface test program (tests/host/test_host, built by
__graft_entry__.build() or `make -C tests/host`)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "host", "test_host")


def run(mode, timeout):
    if not os.path.exists(BINARY):
        raise FileNotFoundError(f"{BINARY} is not built: run __graft_entry__.build() or make -C tests/host")
    p = subprocess.run([BINARY, mode], capture_output=True, text=True, timeout=timeout)
    print(p.stdout)
    print(p.stderr)
    failed = [ln for ln in p.stdout.splitlines() if ln.startswith("[ FAILED ]")]
    assert p.returncode == 0 and not failed, f"host interface cases failed: {failed}\n{p.stdout[-4000:]}"
    return p.stdout
