"""INTEGRATION.md's binding compiles as written.

The C blocks of INTEGRATION.md are compiled, in order, against the reference's
own include/ headers and include/qr_dropin.h / qr_hip.h, each in the reference
source file it belongs to (src/kernels.c, src/runtime.c, src/model.c), with
-std=c99 -Wall -Werror, both with and without -DQR_GPU; every qr_* symbol the
objects use must be exported by libqr_hip.so.  The preludes stand for what
those reference files already define above the edited lines (their static
kernel tables, dot_ref / rmsnorm_ref, ggml_type_row_size); the binding itself
is compiled exactly as documented.  Needs the reference checkout (this
container); skipped elsewhere.
"""
import os
import re
import subprocess

import pytest

import quantr_amd as Q

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/include"

PRELUDES = {
    "kernels": """
#include <string.h>
#include "kernels.h"
static float dot_ref(const float* a, const float* b, int n) {
    float s = 0.0f; int i; for (i = 0; i < n; i++) s += a[i] * b[i]; return s;
}
static void rmsnorm_ref(float* o, const float* x, const float* w, int n) {
    int i; for (i = 0; i < n; i++) o[i] = x[i] * w[i];
}
static void matmul_ref(float* o, const float* x, const float* w, int n, int d, int t) {
    (void)o; (void)x; (void)w; (void)n; (void)d; (void)t;
}
static void softmax_ref(float* x, int n) { (void)x; (void)n; }
static const KernelOps REF_OPS = {matmul_ref, dot_ref, rmsnorm_ref, softmax_ref, "ref"};
static const KernelOps AVX2_OPS = {matmul_ref, dot_ref, rmsnorm_ref, softmax_ref, "avx2"};
static const KernelOps AVX512_OPS = {matmul_ref, dot_ref, rmsnorm_ref, softmax_ref, "avx512"};
""",
    "runtime": """
#include <string.h>
#include "runtime.h"
#include "model.h"
#include "quant.h"
""",
    "model": """
#include "model.h"
#include "quant.h"
static size_t ggml_type_row_size(uint32_t type, size_t ne0) {
    return type == 12 ? (ne0 / 256) * 144 : ne0 * 4;
}
""",
}
# INTEGRATION.md's C blocks, in order, and the reference file each edits
FILES = ["kernels", "runtime", "runtime", "model", "runtime"]


def _blocks():
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    return re.findall(r"```c\n(.*?)```", text, flags=re.S)


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", Q.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


@pytest.mark.skipif(not os.path.isdir(REF_INC), reason="needs the reference's include/")
@pytest.mark.parametrize("gpu", [True, False])
def test_integration_snippets_compile(tmp_path, gpu):
    blocks = _blocks()
    assert len(blocks) == len(FILES), "INTEGRATION.md has %d C blocks" % len(blocks)
    units = {}
    for f, b in zip(FILES, blocks):
        units.setdefault(f, PRELUDES[f])
        units[f] += "\n" + b
    exported = _exported()
    for f, src in units.items():
        c = tmp_path / ("%s.c" % f)
        o = tmp_path / ("%s.o" % f)
        c.write_text(src)
        cmd = ["gcc", "-std=c99", "-O1", "-Wall", "-Wextra", "-Werror", "-Wno-unused-function",
               "-Wno-unused-parameter", "-I", REF_INC, "-I", os.path.join(REPO, "include"),
               "-c", str(c), "-o", str(o)]
        if gpu:
            cmd.insert(1, "-DQR_GPU")
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, "%s.c:\n%s" % (f, r.stderr)
        und = subprocess.run(["nm", "-u", str(o)], capture_output=True, text=True,
                             check=True).stdout.split()
        used = {s for s in und if s.startswith("qr_")}
        assert used <= exported, sorted(used - exported)
        if gpu:
            assert used, "%s.c uses no qr_* symbol" % f
