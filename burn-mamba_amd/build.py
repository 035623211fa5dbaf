"""Build libmamba_hip.so (the gfx950 C-ABI library) in-tree.

    python burn-mamba_amd/build.py          # incremental
    python burn-mamba_amd/build.py --force  # rebuild everything

Each csrc/*.hip file is compiled with hipcc for gfx950 only, then linked into
burn-mamba_amd/lib/libmamba_hip.so.  Packed-f32 VALU ops are disabled
(-packed-fp32-ops) for every device pass.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(LIBDIR, "obj")
LIB = os.path.join(LIBDIR, "libmamba_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]
# per-file additions: MFMA results kept in VGPRs (no AGPR round trips for
# kernels that post-process accumulators with VALU work)
FILE_FLAGS = {
    "ssd2_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "ssd3_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "mamba3_fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the decode products: accumulators in VGPRs keep a wave within 128
    # registers (four waves per SIMD)
    "lin.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


# kernels whose memory waits are hand-counted (an explicit s_waitcnt vmcnt(n)
# with n > 0 after direct-to-LDS loads): a scratch access added by the compiler
# would make the count retire too early, so a build of them with scratch is
# refused.  Checked from the compiler's kernel-resource-usage remarks.
NO_SCRATCH = {
    "mamba1.hip": ("mamba1_scan_tm16",),
}


def _check_no_scratch(src: str, stderr: str) -> None:
    kernels = NO_SCRATCH.get(os.path.basename(src), ())
    cur = None
    seen = set()
    for ln in stderr.splitlines():
        if "Function Name:" in ln:
            cur = next((k for k in kernels if k in ln), None)
        elif cur and "ScratchSize [bytes/lane]:" in ln:
            size = int(ln.split("ScratchSize [bytes/lane]:")[1].split()[0])
            if size != 0:
                raise RuntimeError(f"{cur} in {src} uses {size} bytes/lane of scratch; "
                                   "its hand-counted memory waits assume none")
            seen.add(cur)
    missing = set(kernels) - seen
    if missing:
        raise RuntimeError(f"no resource-usage remark for {sorted(missing)} in {src}")


def _deps_newer(obj: str, src: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + glob.glob(os.path.join(CSRC, "*.h")) + [os.path.join(HERE, "..", "include", "mamba_hip.h")]
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _compile(src: str, force: bool) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src).replace(".hip", ".o"))
    if force or _deps_newer(obj, src):
        check = os.path.basename(src) in NO_SCRATCH
        cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(os.path.basename(src), []),
               *(["-Rpass-analysis=kernel-resource-usage"] if check else []), "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
        if check:
            _check_no_scratch(src, r.stderr or "")
            r.stderr = "\n".join(ln for ln in (r.stderr or "").splitlines()
                                  if "kernel-resource-usage" not in ln and not ln.lstrip().startswith(("|", "^"))
                                  and not ln.lstrip()[:1].isdigit())
        # the host pass does not know the gfx feature flag: that warning is expected
        noise = "'-packed-fp32-ops' is not a recognized feature"
        msgs = [ln for ln in (r.stderr or "").splitlines() if noise not in ln and ln.strip()]
        if msgs:
            sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(force: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    if force or not os.path.exists(LIB) or any(os.path.getmtime(o) > os.path.getmtime(LIB) for o in objs):
        tmp = LIB + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
