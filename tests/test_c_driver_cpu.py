"""The whole-graph generator with the reference front end linked (tests/c_api/tkm_c_driver.c,
built in the build container by oracle/Makefile, target `driver`): the pointwise ops' code
as the registry holds it is pasted into the generated kernels (mode 1, the default), this
build's own formulas are used instead (mode 0), or every pointwise op goes through the path
an op unknown to this build takes (mode 2, TKM_OP_FORMULA*).  All three sources compile with
hipRTC for gfx950."""
import os
import subprocess

import pytest

from tokamak_amd import prep

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER = os.path.join(os.path.dirname(HERE), "oracle", "_ref", "tkm_c_driver")
MODEL = os.path.join(HERE, "golden", "models", "pointwise_mix.tkm")

pytestmark = pytest.mark.skipif(not os.path.exists(DRIVER),
                                reason="oracle/_ref/tkm_c_driver is built only where the reference sources exist")


def _source(mode):
    r = subprocess.run([DRIVER, "source", str(mode), MODEL, "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_generated_source_compiles(mode):
    src = _source(mode)
    rc, code, log = prep.rtc_compile(prep.prelude() + "\n" + src, f"pointwise_mix_{mode}.hip")
    assert rc == 0, log
    assert len(code) > 0


def test_registry_code_is_pasted():
    own, reg, unknown = _source(0), _source(1), _source(2)
    # the registry's code names its parameter-gradient accumulator acc_dw / acc_db; this
    # build's formulas do not
    assert "acc_dw" not in own and "acc_dw" in reg and "acc_db" in reg
    assert "the registry's code of this op" in reg
    # mode 2 maps every pointwise op onto the Formula ops and pastes the same code
    assert "FormulaW" in unknown and "FormulaB" in unknown and "Formula " in unknown
    strip = lambda s: [ln for ln in s.splitlines() if "/* node" not in ln]
    assert strip(reg) == strip(unknown)
