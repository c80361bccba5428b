"""CPU: the tuned-table reading of testt_amd/blas.py (the hipBLASLt solution of each listed GEMM,
keyed as TunableOp keys it) and the C ABI's argument checks of soupk_gemm_lt (no launch)."""

import pytest

from testt_amd import _ext, blas, gemm_tuning


def test_committed_table_keys():
    n = blas.load_table(gemm_tuning.RESULTS)
    try:
        t = dict(blas._table)
        assert n == len(t) and n > 0
        # the layer's gate|up forward (x [2048, 1536] @ W [17920, 1536]^T, column-major
        # m = 17920, n = 2048, k = 1536) and the q|k|v forward with its bias
        assert t[("tn", 17920, 2048, 1536, 1536, 1536, 17920, False)] == 625108
        assert t[("tn", 2048, 2048, 1536, 1536, 1536, 2048, True)] == 624996
        # an input gradient (dy [2048, 2048] @ W [2048, 1536])
        assert t[("nn", 1536, 2048, 2048, 1536, 2048, 1536, False)] == 624622
        # 'Default' rows keep the heuristic: not listed
        assert ("nt", 1536, 32, 2048, 1536, 32, 1536, False) not in t
    finally:
        blas.clear_table()
    assert not blas._table


def test_table_skips_other_rows(tmp_path):
    p = tmp_path / "t.csv"
    p.write_text("Validator,PT_VERSION,x\n"
                 "GemmTunableOp_Half_TN,tn_8_16_32_ld_32_32_8,Gemm_Hipblaslt_7,0.1\n"
                 "GemmTunableOp_Half_NN,nn_8_16_32_ld_8_32_8,Default,0.1\n"
                 "GemmTunableOp_Float_TN,tn_8_16_32_ld_32_32_8,Gemm_Hipblaslt_9,0.1\n"
                 "GemmTunableOp_Half_TN,bad_signature,Gemm_Hipblaslt_5,0.1\n")
    try:
        assert blas.load_table(str(p)) == 1
        assert blas._table == {("tn", 8, 16, 32, 32, 32, 8, False): 7}
    finally:
        blas.clear_table()


@pytest.mark.parametrize("args", [
    (2, 0, 8, 8, 8, 16, 8, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1, None, 0, None),  # trans 2
    (0, 0, 8, 8, 8, 16, 4, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1, None, 0, None),  # lda < m
    (1, 0, 8, 8, 16, 16, 8, 0, 16, 16, 0, 16, 8, 0, 0, 1, 0, None, -1, None, 0, None),  # lda < k
    (0, 0, 8, 8, 8, 16, 8, 0, 16, 8, 0, 16, 8, 0, 0, 0, 0, None, -1, None, 0, None),  # batch 0
    (0, 0, 8, 8, 0, 16, 8, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1, None, 0, None),  # k 0
    (0, 0, 8, 8, 8, 16, 8, 64, 16, 8, 64, 16, 8, 32, 0, 2, 0, None, -1, None, 0, None),  # D overlap
    (0, 0, 8, 8, 8, 16, 8, 0, 16, 8, 0, 16, 8, 0, 1, 1, 0, 16, -1, None, 0, None),  # bias, fp32 D
    (0, 0, 8, 8, 8, None, 8, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1, None, 0, None),  # null A
])
def test_gemm_lt_rejects_before_any_call(args):
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_lt", *args)


def test_gemm_lt_empty_problem_is_a_no_op():
    _ext.call("soupk_gemm_lt", 0, 0, 0, 8, 8, None, 8, 0, None, 8, 0, None, 8, 0, 0, 1, 0, None,
              -1, None, 0, None)
