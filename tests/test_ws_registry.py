"""The workspace registry's rules on the CPU (ws_registry.h with a counting
malloc allocator in place of the device pool): reuse and growth, no buffer
shared by two live threads, and buffers of ended threads adopted by later
ones, so 200 short-lived threads leave as many workspaces as 4 threads alive
at once need, and releasing the streams returns the count to zero."""
import os
import subprocess
import tempfile

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_workspaces_do_not_grow_with_thread_churn():
    src = os.path.join(REPO, "tests", "ws_registry_check.cpp")
    inc = os.path.join(REPO, "sneppx-alg_amd", "csrc")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "ws_check")
        subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-fsanitize=thread", "-I", inc, src, "-o", exe],
                       check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "ok:" in r.stdout
