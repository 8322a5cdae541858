"""`anvil export --hip` (the reference's export.py:68-161 for the HIP backend): a lowered function
as lib<name>.so plus a header with the reference's prototype and SIZE macros. The CPU tests check
the header and that the library exports the entry point; the GPU test links a C program against the
library (built by __graft_entry__.build()) and compares its results with the reference's."""
import os
import subprocess

import numpy as np
import pytest

from fixtures import ROOT, vectors

EXPORT_DIR = os.path.join(ROOT, "anvil-lang_amd", "anvil", "_libs", "export")
HEADER = os.path.join(EXPORT_DIR, "linear_lib.h")
LIB = os.path.join(EXPORT_DIR, "liblinear_lib.so")

APP = r"""
#include <stdio.h>
#include <stdlib.h>
#include "linear_lib.h"
static void readf(const char *path, float *p, size_t n) {
    FILE *f = fopen(path, "rb");
    if (!f || fread(p, sizeof(float), n, f) != n) { fprintf(stderr, "read %s\n", path); exit(2); }
    fclose(f);
}
int main(int argc, char **argv) {
    static float x[LINEAR_LIB_LINEAR_X_SIZE], W[LINEAR_LIB_LINEAR_W_SIZE], b[LINEAR_LIB_LINEAR_B_SIZE];
    static float out[LINEAR_LIB_LINEAR_OUT_SIZE];
    readf(argv[1], x, LINEAR_LIB_LINEAR_X_SIZE);
    readf(argv[2], W, LINEAR_LIB_LINEAR_W_SIZE);
    readf(argv[3], b, LINEAR_LIB_LINEAR_B_SIZE);
    linear_lib_linear(x, W, b, out);
    FILE *f = fopen(argv[4], "wb");
    fwrite(out, sizeof(float), LINEAR_LIB_LINEAR_OUT_SIZE, f);
    fclose(f);
    return 0;
}
"""


def _built():
    if not (os.path.exists(HEADER) and os.path.exists(LIB)):
        pytest.skip("run __graft_entry__.build() first (it exports c3_linear_small)")


def test_export_header_has_the_reference_form():
    _built()
    h = open(HEADER).read()
    assert "void linear_lib_linear(const float *x, const float *W, const float *b, float *out);" in h
    assert "#define LINEAR_LIB_LINEAR_X_SIZE 7680   /* f32[96, 80] */" in h
    assert "#define LINEAR_LIB_LINEAR_W_SIZE 5760   /* f32[72, 80] */" in h
    assert "#define LINEAR_LIB_LINEAR_OUT_SIZE 6912   /* f32[96, 72] */" in h
    assert 'extern "C" {' in h and "#include <stdint.h>" in h


def test_export_library_exports_the_entry_point():
    _built()
    r = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    names = {line.split()[-1] for line in r.stdout.splitlines() if line.strip()}
    assert "linear_lib_linear" in names and "anvil_entry" in names


@pytest.mark.gpu
def test_gpu_exported_library_called_from_c(tmp_path):
    _built()
    print("gpu export linear_lib", flush=True)
    z = vectors("c3_linear_small")
    app = tmp_path / "app.c"
    app.write_text(APP)
    exe = str(tmp_path / "app")
    r = subprocess.run(["gcc", str(app), f"-I{EXPORT_DIR}", f"-L{EXPORT_DIR}", "-llinear_lib",
                        f"-Wl,-rpath,{EXPORT_DIR}", "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    paths = []
    for k in range(3):
        p = tmp_path / f"in{k}.bin"
        np.ascontiguousarray(z[f"input{k}"], dtype=np.float32).tofile(p)
        paths.append(str(p))
    out = tmp_path / "out.bin"
    r = subprocess.run([exe] + paths + [str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(out, dtype=np.float32).reshape(z["output0"].shape)
    want = z["output0"]
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))
