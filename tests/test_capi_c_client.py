"""The C ABI as a plain C caller sees it (CPU only): a C11 program compiled
with gcc against include/spmm_capi.h and linked to libspmm_amd.so, calling
host-side entry points — the reference's uniform generator (csr.cu:74-103;
its committed nnz for 4096^2, density 0.01, seed 42 is 167686), the hybrid
rule (spmm_hybrid.cu:32-56), the host free that zeroes the struct, an error
that comes back as a status with a message instead of exiting, and
spmm_c_unified, spmm_c_hybrid_choose and spmm_c_hybrid_run refusing a matrix
without row_ptr before reading it or calling the device."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "sparse-matrix-multiplication_amd", "build")

CLIENT = r"""
#include <stdio.h>
#include <string.h>
#include "spmm_capi.h"

int main(void) {
    spmm_csr_t a;
    memset(&a, 0, sizeof a);
    if (spmm_c_generate_uniform_random_csr(4096, 4096, 0.01f, 42, &a) != SPMM_OK) {
        printf("generate failed: %s\n", spmm_c_last_error());
        return 1;
    }
    int monotone = a.row_ptr[0] == 0 && a.row_ptr[a.num_rows] == a.nnz;
    for (int r = 0; r < a.num_rows; ++r) monotone &= a.row_ptr[r] <= a.row_ptr[r + 1];
    spmm_hybrid_plan_t p;
    const int rc = spmm_c_hybrid_choose(&a, 128, -1.0f, &p);
    printf("nnz=%d monotone=%d choose_rc=%d backend=%s fill=%.4f reason_set=%d\n", a.nnz,
           monotone, rc, spmm_c_backend_name(p.backend), p.fill_in_ratio,
           p.reason != NULL && p.reason[0] != '\0');
    spmm_c_csr_free_host(&a);
    printf("freed rows=%d nnz=%d null=%d\n", a.num_rows, a.nnz,
           a.row_ptr == NULL && a.col_idx == NULL && a.values == NULL);
    spmm_csr_t bad;
    memset(&bad, 0, sizeof bad);
    const int bad_rc = spmm_c_generate_uniform_random_csr(-1, 4, 0.5f, 1, &bad);
    printf("bad_rc=%d message=%d version=%d\n", bad_rc, spmm_c_last_error()[0] != '\0',
           spmm_c_version()[0] != '\0');
    /* spmm_unified with a missing row_ptr: refused before any device call */
    spmm_csr_t hole;
    memset(&hole, 0, sizeof hole);
    hole.num_rows = 4;
    hole.num_cols = 4;
    float b[16] = {0}, c[16];
    float ms = -1.0f;
    int residency = 7;
    const int un_rc = spmm_c_unified(&hole, b, c, 4, 0, 1, &ms, &residency);
    printf("unified_rc=%d invalid=%d untouched=%d\n", un_rc, un_rc == SPMM_INVALID,
           ms == -1.0f && residency == 7);
    /* the same matrix through the hybrid's choice and run */
    spmm_hybrid_plan_t hp;
    memset(&hp, 0, sizeof hp);
    const int ch_rc = spmm_c_hybrid_choose(&hole, 4, -1.0f, &hp);
    hp.backend = SPMM_BACKEND_CSR;
    const int hy_rc = spmm_c_hybrid_run(&hp, &hole, b, c, 4, 0, 1, &ms);
    printf("choose_invalid=%d run_invalid=%d untouched=%d\n", ch_rc == SPMM_INVALID,
           hy_rc == SPMM_INVALID, ms == -1.0f);
    return 0;
}
"""


def test_c11_client_links_and_runs(S, tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "client.c"
    src.write_text(CLIENT)
    exe = tmp_path / "client"
    cmd = [gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           str(src), "-L", BUILD, "-lspmm_amd", f"-Wl,-rpath,{BUILD}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert lines[0].startswith("nnz=167686 monotone=1 choose_rc=0 backend=csr ")
    assert "reason_set=1" in lines[0]
    fill = float(lines[0].split("fill=")[1].split()[0])
    assert fill == pytest.approx(92.5616, abs=1e-3)  # bench.py's c1 fill-in
    assert lines[1] == "freed rows=0 nnz=0 null=1"
    bad = dict(kv.split("=") for kv in lines[2].split())
    assert bad["bad_rc"] != "0" and bad["message"] == "1" and bad["version"] == "1"
    unified = dict(kv.split("=") for kv in lines[3].split())
    assert unified["invalid"] == "1" and unified["untouched"] == "1", lines[3]
    assert lines[4] == "choose_invalid=1 run_invalid=1 untouched=1", lines[4]
