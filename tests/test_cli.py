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
    r = run("--prompt", "hello")                  # a text prompt needs --model
    assert r.returncode == 2 and "usage" in r.stderr
    r = run("--model", "m.gguf", "--chat")        # --chat needs a prompt
    assert r.returncode == 2
    r = run("--model", "m.gguf", "--prompt-file", "/nonexistent/prompt.txt")
    assert r.returncode == 2 and "cannot open" in r.stderr


def test_cli_verify_cache(xh, tmp_path):
    """--verify-cache (decode.cpp:2580-2661) through the C++ Model class: PASS
    on a fresh cache, FAIL once a payload byte is flipped; no GPU involved."""
    import gguf_util as G
    X = xh
    model = str(tmp_path / "m.gguf")
    G.gemma_model(model, n_layers=1, hidden=256, ffn=512, n_heads=1, vocab=512)
    g = X.Gguf(model)
    cfg = g.config(X.XpConfig.gemma3_1b(scale_fmt=X.XP_SCALE_BF16_QUAD))
    g.pack_model(cfg, model + ".xpack")
    g.close()
    r = run("--model", model, "--layers", 1, "--verify-cache", "--pack-threads", 2)
    assert r.returncode == 0 and "PASS" in r.stdout, r.stdout + r.stderr
    r = run("--model", model, "--pack-cache", model + ".other", "--verify-cache")
    assert r.returncode == 1 and "no valid cache" in r.stderr
    data = bytearray(open(model + ".xpack", "rb").read())
    data[1000] ^= 1
    open(model + ".xpack", "wb").write(bytes(data))
    r = run("--model", model, "--layers", 1, "--verify-cache")
    assert r.returncode == 1 and "FAIL" in r.stdout, r.stdout + r.stderr
    r = run("--verify-cache")
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
        r = run("--layers", layers, "--prompt-len", prompt_len, "-n", n, "--weights-seed", seed,
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


@pytest.mark.gpu
def test_gpu_cli_token_kernel_after_in_process_session(xp):
    """A child process on the same GPU runs the persistent token kernel while
    this process holds a token-kernel session that has launched: the launch
    is a plain one, so nothing is refused and AUTO picks the token kernel in
    both; the ids agree."""
    X = xp
    print("case cli after in-process token session", flush=True)
    seed, layers = 0x5EED0003, 3
    cfg = X.XpConfig.gemma3_1b(n_layers=layers, exec_mode=X.XP_EXEC_AUTO)
    sess = X.DecodeSession(cfg)
    assert sess.exec_mode == X.XP_EXEC_TOKEN
    sess.synthesize(seed)
    sess.prefill(np.array([1, 2, 3], np.uint32))
    sess.decode_steps(4)
    r = run("--layers", layers, "--prompt-len", 8, "-n", 6, "--weights-seed", seed, "--ids")
    assert r.returncode == 0, r.stderr
    assert "persistent token kernel" in r.stdout, r.stdout
    r2 = run("--layers", layers, "--prompt-len", 8, "-n", 6, "--weights-seed", seed, "--ids",
             "--exec", "graph")
    assert r2.returncode == 0, r2.stderr
    assert cli_ids(r.stdout) == cli_ids(r2.stdout)
    sess.decode_steps(2)                  # this process's session still runs
    sess.close()


@pytest.mark.gpu
def test_gpu_cli_gguf_matches_python_session(xp, tmp_path):
    """--model: the CLI's C++ GGUF load (DecodeSession(Model, Config, cache))
    and the Python binding's give the same greedy ids on a small GGUF model."""
    import ctypes as C
    import gguf_util as G
    X = xp
    print("case cli gguf", flush=True)
    model = str(tmp_path / "m.gguf")
    G.gemma_model(model, n_layers=2, hidden=256, ffn=512, n_heads=1, vocab=1024, seed=31)
    seed, prompt_len, n = 0x5EED0003, 4, 6
    r = run("--model", model, "--prompt-len", prompt_len, "-n", n, "--weights-seed", seed, "--ids")
    assert r.returncode == 0, r.stderr
    assert "cache written" in r.stdout, r.stdout
    ids = cli_ids(r.stdout)
    r2 = run("--model", model, "--prompt-len", prompt_len, "-n", n, "--weights-seed", seed,
             "--ids")
    assert r2.returncode == 0 and "from the pack cache" in r2.stdout, r2.stdout + r2.stderr
    assert cli_ids(r2.stdout) == ids
    prompt = []
    for i in range(prompt_len):
        c = (C.c_uint32 * 4)(i, 0, 0, 0)
        k = (C.c_uint32 * 2)(seed, 0x7000)
        o = (C.c_uint32 * 4)()
        X.lib().xp_philox4x32_10(c, k, o)
        prompt.append(o[0] % 1024)
    g = X.Gguf(model)
    cfg = g.config(X.XpConfig.gemma3_1b(scale_fmt=X.XP_SCALE_BF16_QUAD))
    sess = X.DecodeSession(cfg)
    sess.load_gguf(g)
    sess.prefill(np.array(prompt, np.uint32))
    assert [sess.decode_step() for _ in range(n)] == ids
    sess.close()
    g.close()


@pytest.mark.gpu
def test_gpu_cli_text_chat(xp, tmp_path):
    """--text / --chat: the prompt goes through the model's tokenizer (BOS,
    the turn template), and the ids the CLI generates equal the Python
    session's on the same encoded prompt."""
    import gguf_util as G
    X = xp
    print("case cli text", flush=True)
    model = str(tmp_path / "m.gguf")
    G.gemma_model(model, n_layers=2, hidden=256, ffn=512, n_heads=1, vocab=1024, seed=41, chat=True)
    pf = tmp_path / "prompt.txt"
    pf.write_bytes(b"hello world")
    r = run("--model", model, "--no-pack-cache", "--prompt-file", pf, "--chat", "-n", 6, "--ids")
    assert r.returncode == 0, r.stderr
    assert "<start_of_turn>user\nhello world<end_of_turn>" in r.stdout
    ids = cli_ids(r.stdout)
    g = X.Gguf(model)
    tok = X.Tokenizer(g)
    prompt = tok.encode("<start_of_turn>user\nhello world<end_of_turn>\n<start_of_turn>model\n",
                        add_bos=True)
    assert prompt[0] == 2 and prompt[1] == 4          # <bos> <start_of_turn>
    cfg = g.config(X.XpConfig.gemma3_1b(scale_fmt=X.XP_SCALE_BF16_QUAD))
    sess = X.DecodeSession(cfg)
    sess.load_gguf(g)
    sess.prefill(np.array(prompt, np.uint32))
    got = []
    for _ in range(6):
        t = sess.decode_step()
        if t in (1, 5):                               # <eos>, <end_of_turn>
            break
        got.append(t)
    assert got == ids
    tok.close()
    sess.close()
    g.close()
