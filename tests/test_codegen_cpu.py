"""Instruction-selection guards on the gfx950 device code (CPU: hipcc -S only).

Two instruction forms have given wrong results on the MI355X boxes this
library runs on, silently:
  * packed FP32 VALU ops (v_pk_add/mul/fma_f32): the build disables them
    (-packed-fp32-ops); this checks that the flag took effect;
  * a mixed-precision FMA (v_fma_mix*/v_mad_mix*) with a negated operand: the
    hi/lo split of q (pa_common.h split_f16x8) was compiled to one and came out
    as hi - x instead of x - hi (caught by the peaked-score parity tests); the
    source keeps the compiler from forming it.
It also checks that the prefill kernels' lo product of q runs on the scaled
fp8 MFMA with both operands in bf8 (OCP E5M2, format code 1: cbsz:1 blgp:1),
the format whose encoding is the top byte of an f16 (pa_mfma.h).
"""
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from iian_amd import build as B

# every device source of the library (pa_abi.hip is host code only)
KERNEL_SOURCES = [s for s in B.SOURCES if s not in ("pa_abi.hip", "pa_runtime.hip")]   # host code only
NO_MFMA = {"pa_kv_write.hip", "pa_general.hip", "pa_batch.hip", "pa_rope.hip"}
PACKED_F32 = re.compile(r"^\s*v_pk_(add|mul|fma)_f32\b", re.M)
NEG_MIX = re.compile(r"^\s*v_(fma|mad)_mix\w*\s[^\n]*,\s*-", re.M)


def device_asm(src: str, tmp: Path) -> str:
    out = tmp / (Path(src).stem + ".s")
    cmd = [B.hipcc(), *B.HIPCC_FLAGS, "--cuda-device-only", "-S", str(B.CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_no_packed_fp32_and_no_negated_mixed_fma(tmp_path):
    with ThreadPoolExecutor(len(KERNEL_SOURCES)) as ex:
        asms = dict(zip(KERNEL_SOURCES, ex.map(lambda s: device_asm(s, tmp_path), KERNEL_SOURCES)))
    for src, asm in asms.items():
        assert "v_mfma" in asm or src in NO_MFMA, src   # the asm is the kernels'
        assert not PACKED_F32.search(asm), (src, PACKED_F32.search(asm).group(0))
        m = NEG_MIX.search(asm)
        assert m is None, (src, m.group(0) if m else None)


BF8_LO = re.compile(r"^\s*v_mfma_scale_f32_(32x32x64|16x16x128)_f8f6f4\s[^\n]*$", re.M)


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_prefill_lo_product_is_bf8(tmp_path):
    for src, shape in (("pa_prefill.hip", "32x32x64"), ("pa_prefill16.hip", "16x16x128")):
        lines = [m.group(0) for m in BF8_LO.finditer(device_asm(src, tmp_path))]
        assert any(shape in l for l in lines), src
        for l in lines:
            assert "cbsz:1" in l and "blgp:1" in l, (src, l)
