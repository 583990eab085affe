"""`python -m simd_ml_kernels selftest` (the reference's selftest command, _cli.py:324-348, for the
single gfx950 table): the CPU side checks the command line and the check list, the GPU side runs
every check and requires all of them to pass within their bounds."""

import contextlib
import io

import pytest


def test_info_and_check_list():
    from simd_ml_kernels import __main__ as cli
    out = io.StringIO()
    with contextlib.redirect_stdout(out):
        assert cli.main(["info"]) == 0
    assert "isa_compiled: gfx950" in out.getvalue()
    names = [n for n, _ in cli.selftest_checks()]
    for kernel in ("x quantizer", "gemv_q4_0", "gemv_q8_0", "sgemm tb", "sgemm_f16 tb", "sgemm_bf16 tb", "silu",
                   "softmax", "rms_norm", "rope"):
        assert kernel in names
    with pytest.raises(SystemExit):
        cli.main(["no-such-command"])


@pytest.mark.gpu
def test_selftest_passes_on_the_device():
    from simd_ml_kernels import __main__ as cli
    out = io.StringIO()
    with contextlib.redirect_stdout(out):
        rc = cli.main(["selftest"])
    text = out.getvalue()
    print(text)
    assert rc == 0, text
    assert "selftest: passed" in text
    assert text.count("  PASS  ") == len(cli.selftest_checks())
