"""Mutation fuzzing of the GGUF parser and model mapping (host/qr_gguf.c)
under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU: the
reference ships a mutation fuzzer for its parser (tests/fuzz_gguf.c:46-77);
tests/native/gguf_fuzz.c runs its cases (tiny and corrupt headers, random and
magic-prefixed payloads) and structure-aware mutations of valid model files
(MoE and dense, 32- and 64-byte alignment, 3-D and per-expert expert
tensors).  Any sanitizer report fails the run."""
import os
import shutil
import subprocess

import pytest

import gguf_writer as G
import inputs as I

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    out = tmp_path_factory.mktemp("fuzz")
    exe = str(out / "gguf_fuzz")
    cmd = ["gcc", "-O1", "-g", "-std=c99", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           "-I", os.path.join(REPO, "include"),
           os.path.join(REPO, "tests", "native", "gguf_fuzz.c"),
           os.path.join(REPO, "quantr-in-c_amd", "host", "qr_gguf.c"), "-o", exe]
    subprocess.run(cmd, check=True)
    seeds = []
    a, c = I.decode_model("a"), I.decode_model("c")
    q3 = I.qwen3_small_model(n_layers=1, seq_len=64)
    for name, data in (("a", G.decode_model_gguf(a)[0]),
                       ("a64", G.decode_model_gguf(a, alignment=64)[0]),
                       ("c_dense", G.decode_model_gguf(c)[0]),
                       ("q3_split", G.decode_model_gguf(q3, split_experts=True,
                                                        head_dim_key=True)[0])):
        p = out / (name + ".gguf")
        p.write_bytes(data)
        seeds.append(str(p))
    return exe, seeds


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_gguf_mutation_fuzz(fuzzer, seed):
    exe, seeds = fuzzer
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, str(seed), "6000"] + seeds, capture_output=True, text=True,
                       timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, \
        r.stderr[-4000:]
    print(r.stdout.strip())
    # the structure-aware mutations reach the mapping, not only the header checks
    parsed = int(r.stdout.split(" inputs, ")[1].split(" parsed")[0])
    assert parsed > 100
