"""A plain C11 caller running the hot path through the C ABI on the GPU:
spmm_c_hybrid_run (spmm_hybrid.cu:58-125: host in, host out) on a uniform
matrix the rule sends to CSR and on a banded one it sends to the MFMA kernel,
each checked inside the C program against its own fp64 loop over the same
inputs (relative L2 within 1e-6 for CSR, 5e-3 for the fp16 MFMA path)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "sparse-matrix-multiplication_amd", "build")

pytestmark = pytest.mark.gpu

CLIENT = r"""
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "spmm_capi.h"

static double rel_l2(const spmm_csr_t* a, const float* b, const float* c, int n) {
    double num = 0.0, den = 0.0;
    for (int r = 0; r < a->num_rows; ++r) {
        for (int j = 0; j < n; ++j) {
            double s = 0.0;
            for (int p = a->row_ptr[r]; p < a->row_ptr[r + 1]; ++p)
                s += (double)a->values[p] * (double)b[(size_t)a->col_idx[p] * n + j];
            const double d = (double)c[(size_t)r * n + j] - s;
            num += d * d;
            den += s * s;
        }
    }
    return sqrt(num / (den > 0.0 ? den : 1.0));
}

static int run(const char* name, spmm_csr_t* a, int n) {
    float* b = malloc(sizeof(float) * (size_t)a->num_cols * n);
    float* c = malloc(sizeof(float) * (size_t)a->num_rows * n);
    if (b == NULL || c == NULL) return 1;
    if (spmm_c_generate_dense_row_major(a->num_cols, n, 43, b) != SPMM_OK) return 1;
    for (size_t i = 0; i < (size_t)a->num_rows * n; ++i) c[i] = NAN;
    spmm_hybrid_plan_t plan;
    float ms = -1.0f;
    if (spmm_c_hybrid_choose(a, n, -1.0f, &plan) != SPMM_OK ||
        spmm_c_hybrid_run(&plan, a, b, c, n, 1, 3, &ms) != SPMM_OK) {
        printf("%s failed: %s\n", name, spmm_c_last_error());
        return 1;
    }
    printf("%s backend=%s rel_l2=%.3e ms_ok=%d\n", name, spmm_c_backend_name(plan.backend),
           rel_l2(a, b, c, n), ms > 0.0f);
    free(b);
    free(c);
    return 0;
}

int main(void) {
    spmm_csr_t u, k;
    memset(&u, 0, sizeof u);
    memset(&k, 0, sizeof k);
    if (spmm_c_generate_uniform_random_csr(1024, 1024, 0.01f, 42, &u) != SPMM_OK ||
        spmm_c_generate_banded_csr(1024, 1024, 32, 7, &k) != SPMM_OK) {
        printf("generate failed: %s\n", spmm_c_last_error());
        return 1;
    }
    if (run("uniform", &u, 64) || run("banded", &k, 128)) return 1;
    spmm_c_csr_free_host(&u);
    spmm_c_csr_free_host(&k);
    return 0;
}
"""


def test_c11_client_runs_the_hybrid_on_the_gpu(S, tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "client.c"
    src.write_text(CLIENT)
    exe = tmp_path / "client"
    cmd = [gcc, "-std=c11", "-O1", "-Wall", "-Wextra", "-Werror", "-I",
           os.path.join(ROOT, "include"), str(src), "-L", BUILD, "-lspmm_amd",
           f"-Wl,-rpath,{BUILD}", "-lm", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    print("running C client (uniform 1024^2 N=64, banded 1024^2 N=128)", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    got = {}
    for line in r.stdout.splitlines():
        name, *kv = line.split()
        got[name] = dict(x.split("=") for x in kv)
    assert got["uniform"]["backend"] == "csr" and float(got["uniform"]["rel_l2"]) < 1e-6
    assert got["banded"]["backend"] == "wmma" and float(got["banded"]["rel_l2"]) < 5e-3
    assert got["uniform"]["ms_ok"] == "1" and got["banded"]["ms_ok"] == "1"
