"""The C++ host interface (include/xpose.hpp) through the decode CLI,
xpose_amd/cli/xpose_decode.cpp — the counterpart of the reference's decode
CLI (examples/llm/decode.cpp:2720-3006)."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "xpose_amd", "bin", "xpose_decode")


def run(*args, timeout=120):
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_cli_usage_errors_exit_2():
    """Argument errors are reported before any device is touched."""
    assert os.path.exists(CLI), "build() builds xpose_amd/bin/xpose_decode"
    r = run("--exec", "vulkan")
    assert r.returncode == 2 and "usage" in r.stderr
    r = run("--no-such-flag")
    assert r.returncode == 2


def cli_ids(out: str):
    line = [l for l in out.splitlines() if l.startswith("ids ")][0]
    return [int(t) for t in line.split()[1:]]


@pytest.mark.gpu
def test_gpu_cli_matches_python_session(xp):
    """Same synthetic model and prompt through the C++ class and through the
    Python binding; both executions of the token step give the same ids."""
    import ctypes as C
    X = xp
    print("case cli decode", flush=True)
    seed, layers, prompt_len, n = 0x5EED0003, 3, 8, 12
    outs = {}
    for mode in ("token", "graph"):
        r = run("--layers", layers, "--prompt", prompt_len, "--tokens", n, "--seed", seed,
                "--exec", mode, "--ids")
        assert r.returncode == 0, r.stderr
        outs[mode] = cli_ids(r.stdout)
    assert outs["token"] == outs["graph"]
    # The CLI's prompt: Philox4x32-10 stream (seed, 0x7000), counter i, word 0.
    prompt = []
    for i in range(prompt_len):
        c = (C.c_uint32 * 4)(i, 0, 0, 0)
        k = (C.c_uint32 * 2)(seed, 0x7000)
        o = (C.c_uint32 * 4)()
        X.lib().xp_philox4x32_10(c, k, o)
        prompt.append(o[0] % 262144)
    cfg = X.XpConfig.gemma3_1b(n_layers=layers)
    sess = X.DecodeSession(cfg)
    sess.synthesize(seed)
    sess.prefill(np.array(prompt, np.uint32))
    got = [sess.decode_step() for _ in range(n)]
    assert got == outs["token"]
