"""The host planners (kvc_decode_plan, kvc_prefill_plan) under AddressSanitizer
and UndefinedBehaviorSanitizer, on the CPU: tests/native/plan_fuzz.cpp plans
2000 random batches (empty requests, 0-40000-token contexts, head counts,
group sizes, head dims, forced segment counts, too-small plan buffers that
must be retried at the reported capacity) and checks every plan image against
the invariants the kernels rely on.  The library sources are compiled with
the sanitizers on their host side only (-Xarch_host); no GPU is used."""
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from gpu_offloading_amd.build import ARCH, CSRC, INCLUDE, hipcc

HERE = os.path.dirname(os.path.abspath(__file__))
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all"]


def _run(cmd):
    return subprocess.run(cmd, capture_output=True, text=True)


def test_host_planners_under_sanitizers(tmp_path):
    flags = [f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", *SANITIZE,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             f"-I{INCLUDE}", f"-I{CSRC}"]
    srcs = [os.path.join(CSRC, f) for f in ("api.hip", "decode.hip", "prefill.hip")]
    objs = [str(tmp_path / (os.path.basename(s)[:-4] + ".o")) for s in srcs]
    cmds = [[hipcc(), *flags, "-c", s, "-o", o] for s, o in zip(srcs, objs)]
    fuzz_o = str(tmp_path / "plan_fuzz.o")
    cmds.append([hipcc(), *flags, "-c", "-x", "c++", os.path.join(HERE, "native", "plan_fuzz.cpp"),
                 "-o", fuzz_o])
    with ThreadPoolExecutor(max_workers=4) as ex:
        for res in ex.map(_run, cmds):
            assert res.returncode == 0, res.stderr[-3000:]
    exe = str(tmp_path / "plan_fuzz")
    res = _run([hipcc(), f"--offload-arch={ARCH}", *SANITIZE[:4], *objs, fuzz_o, "-o", exe])
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([exe, "2000"], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0 and res.stdout.strip() == "ok 2000", \
        (res.stdout[-2000:], res.stderr[-4000:])
