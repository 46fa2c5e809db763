"""The GPT-2 engine's tuned GEMM solution file, checked on the CPU."""

def test_gemm_solution_file_is_tunableop_csv_with_validators():
    """The engine's GEMM solution file (dfattn.gpt2_step.GEMM_SOLUTIONS, written by tune_gemms) is a
    TunableOp results file: the library validators first, then one row per GEMM shape naming a
    default, hipBLASLt or rocBLAS solution and its measured time; exact fp32 ("float") ops and fast
    fp32 ("tf32") ops keep their own math mode."""
    from dfattn.gpt2_step import GEMM_SOLUTIONS

    rows = [line.rstrip("\n").split(",") for line in open(GEMM_SOLUTIONS) if line.strip()]
    validators = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    for key in ("PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION", "GCN_ARCH_NAME"):
        assert key in validators, key
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    shapes = [r for r in rows if r[0] != "Validator"]
    assert len(shapes) >= 10
    for op, params, solution, ms in shapes:
        assert "_float_" in op or "_tf32_" in op, op
        assert solution == "Default" or solution.startswith(("Gemm_Hipblaslt_", "Gemm_Rocblas_")), solution
        assert float(ms) > 0
    assert len({(r[0], r[1]) for r in shapes}) == len(shapes)
