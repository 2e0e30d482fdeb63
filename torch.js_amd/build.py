"""Builds libtorchjs_hip.so (gfx950) and the Node-API addon in-tree.

    python torch.js_amd/build.py            # library + addon
    python torch.js_amd/build.py --lib-only
    python torch.js_amd/build.py --changed  # only sources newer than their objects

Every HIP source under csrc/ is compiled by hipcc for gfx950 into
_build/*.o (in parallel) and linked into torch.js_amd/libtorchjs_hip.so.
The Node-API addon (node/torchjs_hip_napi.c) is compiled by gcc against the
system node headers and linked to the library with an $ORIGIN rpath.
"""
import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtorchjs_hip.so")
ADDON_SRC = os.path.join(PKG, "node", "torchjs_hip_napi.c")
ADDON = os.path.join(PKG, "node", "torchjs_hip.node")
INCLUDE = os.path.join(os.path.dirname(PKG), "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM_LIB = "/opt/rocm/lib"
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-I" + INCLUDE,
    # packed fp32 ops are disabled for every HIP translation unit
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the device-only target feature: drop it
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (p.returncode, " ".join(cmd), out))
    return out


def _obj(src):
    return os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))


def _compile(src):
    obj = _obj(src)
    _run([HIPCC] + HIP_FLAGS + ["-c", src, "-o", obj])
    return obj


def _stale(src, headers_mtime):
    obj = _obj(src)
    if not os.path.exists(obj):
        return True
    return os.path.getmtime(obj) < max(os.path.getmtime(src), headers_mtime)


def build_library(jobs=None, changed_only=False):
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources under %s" % CSRC)
    todo = sources
    if changed_only:
        hdrs = glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(INCLUDE, "*.h"))
        hm = max([os.path.getmtime(h) for h in hdrs] or [0.0])
        todo = [s for s in sources if _stale(s, hm)]
    jobs = jobs or min(max(1, len(todo)), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [_obj(s) for s in sources]
    tmp = LIB + ".tmp"
    # roctx (rocprofiler-sdk) for the named ranges of record_function,
    # hipRTC for the fused expression kernels compiled at run time
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs +
         ["-L" + ROCM_LIB, "-lrocprofiler-sdk-roctx", "-lhiprtc", "-Wl,-rpath," + ROCM_LIB])
    os.replace(tmp, LIB)
    return LIB


def build_addon():
    """Node-API addon: plain C against node_api.h, no node-gyp needed."""
    node_inc = "/usr/include/node"
    if not os.path.exists(os.path.join(node_inc, "node_api.h")):
        return None
    cc = shutil.which("gcc") or "cc"
    tmp = ADDON + ".tmp"
    _run([cc, "-O2", "-fPIC", "-shared", "-std=c99", "-I" + node_inc, "-I" + INCLUDE,
          "-DNAPI_VERSION=8", ADDON_SRC, "-o", tmp, "-L" + PKG, "-ltorchjs_hip",
          "-Wl,-rpath,$ORIGIN/.."])
    os.replace(tmp, ADDON)
    return ADDON


def main(argv):
    lib = build_library(changed_only="--changed" in argv)
    print("built", lib)
    if "--lib-only" not in argv and os.path.exists(ADDON_SRC):
        addon = build_addon()
        if addon:
            print("built", addon)


if __name__ == "__main__":
    main(sys.argv[1:])
