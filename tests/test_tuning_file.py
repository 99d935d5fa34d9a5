"""The stack's GEMM tuning file (a TunableOp results file): validator lines
for the libraries it was measured with, and a solution for each of the six
bf16 projection products of a block at the 12-layer configuration's shape."""
import csv

from sparc_amd.stack import GEMM_TUNING_FILE


def test_tuning_file_covers_the_projection_gemms():
    rows = list(csv.reader(open(GEMM_TUNING_FILE)))
    validators = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    for key in ("PT_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION", "GCN_ARCH_NAME"):
        assert key in validators
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    bf16 = {r[1].split("_ld_")[0] for r in rows if r[0].startswith("GemmTunableOp_BFloat16")}
    R, D, W = 16 * 2048, 768, 2 * 768 * 16
    # column-major BLAS problems (op, m, n, k) of the four projections' forward and backward
    want = {f"nn_{W}_{R}_{D}", f"nn_{D}_{R}_{W}", f"tn_{W}_{R}_{D}", f"tn_{D}_{R}_{W}",
            f"nt_{D}_{W}_{R}", f"nt_{W}_{D}_{R}"}
    assert want <= bf16
    for r in rows:
        if r[0] != "Validator":
            assert r[2].startswith(("Gemm_Hipblaslt_", "Gemm_Rocblas_")) and float(r[3]) > 0
