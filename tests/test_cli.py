"""The command-line encoders' argument handling (no GPU work: every case
ends before a model is loaded).  Exit codes as the reference's CLIs
(src/siglip2_cli.cpp, src/siglip2_text_cli.cpp): 0 for --help, 2 for bad
arguments."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "hbd-siglip2.cpp_amd",
                   "bin")


def _run(name, *args):
    exe = os.path.join(BIN, name)
    if not os.access(exe, os.X_OK):
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args,rc,msg", [
    (["--help"], 0, "Usage"),
    (["--bogus"], 2, "Unknown arg"),
    ([], 2, "exactly one of"),
    (["--model", "m.gguf"], 2, "exactly one of"),
    (["--model", "m.gguf", "--pixel-values", "a", "--image", "b"], 2, "exactly one of"),
    (["--model", "m.gguf", "--pixel-values", "a", "--pooling", "max"], 2, "Unknown --pooling"),
    (["--model", "m.gguf", "--pixel-values", "a", "--shape", "27"], 2, "expects H,W"),
    (["--model", "m.gguf", "--rgb", "a"], 2, "--rgb-shape"),
])
def test_vision_cli_arguments(args, rc, msg):
    r = _run("siglip2-cli", *args)
    assert r.returncode == rc and msg in r.stderr, (r.returncode, r.stderr)


@pytest.mark.parametrize("args,rc,msg", [
    (["--help"], 0, "Usage"),
    (["--bogus"], 2, "Unknown arg"),
    ([], 2, "Usage"),
    (["--model", "m.gguf"], 2, "Provide exactly one of"),
    (["--model", "m.gguf", "--token-ids", "a"], 2, "Provide exactly one of"),
    (["--model", "m.gguf", "--token-ids", "a", "--attention-mask", "b", "--tokenizer", "t",
      "--text", "x"], 2, "Provide exactly one of"),
])
def test_text_cli_arguments(args, rc, msg):
    r = _run("siglip2-text-cli", *args)
    assert r.returncode == rc and msg in r.stderr, (r.returncode, r.stderr)
