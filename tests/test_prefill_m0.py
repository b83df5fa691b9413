"""Build-time check of the continuation-prefill kernel's AMD assembly (built
here with hipcc): its direct-to-LDS loads (global_load_lds_dwordx4, buffer_load
... lds) take their LDS address from M0, which the inline assembly writes and
cannot declare clobbered (hipcc reserves M0).  So nothing the compiler
generates may use M0: every instruction naming M0 is one of the kernel's own
M0 writes -- `s_mov_b32 m0, sN` or, between the four loads of one page,
`s_add_u32 m0, m0, 0x400` right after a load -- each directly followed by a
direct-to-LDS load, every such load directly preceded by one, and no
instruction that reads M0 implicitly (relative moves, messages,
interpolation, GWS, append/consume) appears."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"
IMPLICIT_M0 = re.compile(r"^(s_movrel|v_movrel|s_sendmsg|v_interp|ds_gws|ds_append|ds_consume|"
                         r"s_set_gpr_idx|lds_param_load|lds_direct_load)")
LDS_DMA = re.compile(r"^(global_load_lds_\w+ .*|buffer_load_\w+ .* lds)$")


def _instructions(asm: str):
    for line in asm.splitlines():
        code = line.split(";", 1)[0].strip()
        if not code or code.startswith(".") or code.endswith(":"):
            continue
        yield code


@pytest.mark.skipif(not os.access(HIPCC, os.X_OK), reason="hipcc not available")
def test_only_the_direct_lds_loads_use_m0(tmp_path):
    out = tmp_path / "prefill.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-I" + os.path.join(ROOT, "include"),
                    "-I" + os.path.join(ROOT, "gpu_offloading_amd", "csrc"),
                    "--cuda-device-only", "-S",
                    os.path.join(ROOT, "gpu_offloading_amd", "csrc", "prefill.hip"),
                    "-o", str(out)], check=True, capture_output=True)
    ins = list(_instructions(out.read_text()))
    assert ins, "empty assembly"
    set_m0 = re.compile(r"^s_mov_b32 m0, s\d+$")
    step_m0 = re.compile(r"^s_add_u32 m0, m0, 0x400$")
    n_dma = 0
    for i, code in enumerate(ins):
        assert not IMPLICIT_M0.match(code), code
        if LDS_DMA.match(code):
            n_dma += 1
            assert i > 0 and (set_m0.match(ins[i - 1]) or step_m0.match(ins[i - 1])), \
                (ins[i - 1], code)
        if re.search(r"\bm0\b", code):
            assert set_m0.match(code) or step_m0.match(code), code
            if step_m0.match(code):
                assert i > 0 and LDS_DMA.match(ins[i - 1]), (ins[i - 1], code)
            assert i + 1 < len(ins) and LDS_DMA.match(ins[i + 1]), (code, ins[i + 1:i + 2])
    assert n_dma > 0
