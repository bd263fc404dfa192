"""Build the CPU executor library (test infrastructure): the package's HIP sources
compiled as host C++ against emu.h, linked with the executor into
``_build/libsgd_emu[_asan].so``.

The sources are compiled unchanged except for one mechanical rewrite: a dynamic-LDS
declaration ``extern __shared__ [__align__(N)] char NAME[];`` becomes a pointer to the
workgroup's dynamic LDS block (``__shared__`` is ``static`` here, and an extern static
does not exist in C++).  The rewritten copies live under ``_build/`` with the same
relative layout, so the sources' relative includes still resolve.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "-sglang-decode-_amd", "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
CLANG = "/opt/rocm/llvm/bin/clang++"

_DYN_LDS = re.compile(r"extern\s+__shared__\s+(?:__align__\(\d+\)\s+)?char\s+(\w+)\[\];")
_ASM_REG = re.compile(r'asm volatile\(""\s*:\s*"\+[vs]"\((\w+)\)\)')


def asan_runtime():
    """Path of clang's AddressSanitizer runtime (preloaded into the process that loads
    the ASan build)."""
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True, check=True).stdout.strip()
    if not os.path.exists(out):
        import glob
        hits = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
        if not hits:
            raise RuntimeError("clang's ASan runtime not found")
        out = hits[0]
    return out


def lib_path(asan):
    return os.path.join(BUILD, "libsgd_emu_asan.so" if asan else "libsgd_emu.so")


def _stage_sources():
    src_dir = os.path.join(BUILD, "pkg", "csrc")
    inc_dir = os.path.join(BUILD, "include")
    for d in (src_dir, inc_dir):
        shutil.rmtree(d, ignore_errors=True)
        os.makedirs(d)
    shutil.copy(os.path.join(INCLUDE, "sglang_decode_hip.h"), inc_dir)
    staged = []
    for name in sorted(os.listdir(CSRC)):
        if not name.endswith((".hip", ".h")):
            continue
        with open(os.path.join(CSRC, name)) as f:
            text = f.read()
        text = _DYN_LDS.sub(lambda m: f"char *const {m.group(1)} = static_cast<char *>(::emu::dynamic_lds());",
                            text)
        # register-class constraints of the value-laundering asm ("" : "+v"(x)): any
        # operand in memory serves the same purpose on the CPU
        text = _ASM_REG.sub(r'asm volatile("" : "+m"(\1))', text)
        with open(os.path.join(src_dir, name), "w") as f:
            f.write(text)
        if name.endswith(".hip"):
            staged.append(os.path.join(src_dir, name))
    return staged


def build(asan=True, jobs=8, opt="-O1"):
    """Compile every kernel source plus the executor; returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = _stage_sources() + [os.path.join(HERE, "emu.cpp")]
    tag = "asan" if asan else "plain"
    flags = ["-std=c++20", opt, "-g", "-fPIC", "-fno-omit-frame-pointer", "-w",
             "-I", os.path.join(HERE, "include"), "-I", HERE]
    if asan:
        flags += ["-fsanitize=address"]

    def compile_one(src):
        obj = os.path.join(BUILD, f"{os.path.basename(src)}.{tag}.o")
        cmd = [CLANG, "-x", "c++", *flags, "-c", src, "-o", obj]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode:
            raise RuntimeError(f"emu compile failed: {src}\n{p.stdout}\n{p.stderr}")
        return obj

    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(compile_one, srcs))
    out = lib_path(asan)
    cmd = [CLANG, "-shared", *(["-fsanitize=address", "-shared-libasan"] if asan else []), "-o", out + ".tmp",
           *objs]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode:
        raise RuntimeError(f"emu link failed\n{p.stdout}\n{p.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    import sys
    print(build(asan="--plain" not in sys.argv))
