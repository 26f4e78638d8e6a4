"""Instruction guards on the gfx950 device code (CPU only: hipcc cross-compiles).

* No mixed-precision fma (v_fma_mix*, v_mad_mix*).  The compiler forms them
  by fusing an fp32 multiply (or fma) with the fp16 conversion of its result
  (one rounding where the reference rounds twice: fp32 arithmetic, then
  .to(torch.float16)), or by folding an fp16 operand's widening into every
  fma that uses it (v_fma_mix_f32 issues at about half the rate of
  v_fma_f32).  The first breaks the bit-exact contracts of the encode
  (compression.py:287-335), the decoded K/V rows (compression.py:355-359) and
  q_rot (compression.py:290-291); the kernels keep the fp32 value opaque
  before each conversion and widen fp16 operands once.
* No packed fp32 arithmetic (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32): the
  build disables it for all device code.
"""
import re
import shutil
import subprocess

import pytest

from sub0_amd import build as B

FORBIDDEN = re.compile(r"^\s*(v_fma_mix\w*|v_mad_mix\w*|v_pk_fma_f32|v_pk_mul_f32|v_pk_add_f32)\b",
                       re.M)


def _device_asm(src, tmp_path):
    out = tmp_path / (src.stem + ".s")
    flags = [f for f in B.CFLAGS if f not in ("-fPIC",)]
    cmd = [B.HIPCC, *flags, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, f"hipcc failed for {src.name}:\n{r.stderr[-2000:]}"
    return out.read_text()


@pytest.mark.skipif(shutil.which(B.HIPCC) is None, reason="hipcc not available")
@pytest.mark.parametrize("src", B.sources(), ids=lambda p: p.name)
def test_no_mixed_precision_or_packed_fp32(src, tmp_path):
    asm = _device_asm(src, tmp_path)
    hits = FORBIDDEN.findall(asm)
    assert not hits, f"{src.name}: {len(hits)} forbidden instructions, e.g. {sorted(set(hits))[:5]}"
