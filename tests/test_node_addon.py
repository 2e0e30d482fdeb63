"""The Node-API binding (torch.js_amd/node/torchjs_hip_napi.c): the entry
points torch.js's TypeScript host would call for device 'hip'."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "torch.js_amd", "node", "torchjs_hip.node")
CHECK = os.path.join(ROOT, "torch.js_amd", "node", "addon_check.js")
NODE = shutil.which("node")

EXPORTS = ["init", "deviceInfo", "malloc", "h2d", "d2h", "d2hAsync", "synchronize",
           "memoryStats", "emptyCache", "fill", "random", "copyStrided", "unary",
           "unaryBackward", "binary", "scalar", "reduce", "softmaxForward", "softmaxBackward",
           "crossEntropyForward", "crossEntropyBackward", "crossEntropyForwardGrad",
           "layerNormForward",
           "layerNormBackward", "layerNormBackwardRes", "layerNormBackwardNoalloc", "flushDeferred", "embeddingForward", "embeddingBackward",
           "embeddingPosForward", "embeddingPosBackward", "gemm", "gemmAct", "gemmCe", "crossEntropyRowScale",
           "sdpaForward",
           "sdpaBackward", "adamStep", "version", "isInitialized", "deviceCount", "free",
           "resetPeak", "d2d", "kprofEnable", "kprofFilter", "kprofReset", "kprofQuery",
           "kprofNames", "timerStart", "timerStop", "fillI32", "copyStridedI32", "castF32I32",
           "castI32F32", "ternary", "powScalarBackward", "axpy", "maskedFill", "compare",
           "argmax", "nllLossForward", "nllLossBackward", "indexSelect", "indexAdd", "gather",
           "scatterAdd", "oneHot", "oneHotI32", "nonzero", "conv2dForward", "conv2dForwardAct",
           "conv2dBackwardInput", "conv2dBackwardWeight", "conv2dBackwardWeightBias", "cast", "fillU8", "copyStridedU8",
           "triangle", "multinomial", "timerEnd", "timerRead", "rangePush", "rangePop",
           "mark", "exprEval", "exprColsum", "exprColsum2", "exprColsum3", "exprCompile", "graphBegin", "graphEnd", "graphReplay",
           "graphDestroy", "adamStepDev"]
HEADER = os.path.join(ROOT, "include", "torchjs_hip.h")
SOURCE = os.path.join(ROOT, "torch.js_amd", "node", "torchjs_hip_napi.c")

needs_addon = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON),
                                 reason="node or the built addon is absent")


def _node(script, timeout=60):
    return subprocess.run([NODE, "-e", script], capture_output=True, text=True, timeout=timeout,
                          cwd=ROOT)


@needs_addon
def test_addon_exports():
    r = _node("const a=require(%r); console.log(JSON.stringify(Object.keys(a)))" % ADDON)
    assert r.returncode == 0, r.stderr
    keys = json.loads(r.stdout)
    assert sorted(keys) == sorted(EXPORTS)


def test_addon_binds_every_declared_entry_point():
    """Every function the C ABI header declares is called by the addon."""
    import re
    declared = set(re.findall(r"^(?:int|const char\*)\s+(tjh_\w+)\(", open(HEADER).read(),
                              re.M))
    called = set(re.findall(r"(tjh_\w+)\(", open(SOURCE).read()))
    assert declared, "no declarations parsed"
    assert not declared - called, sorted(declared - called)


@needs_addon
def test_addon_error_before_init():
    # no device call happens: the library refuses before touching HIP
    r = _node("const a=require(%r); try { a.synchronize(); console.log('no-throw') } "
              "catch (e) { console.log(e.message) }" % ADDON)
    assert r.returncode == 0, r.stderr
    assert "not initialized" in r.stdout


@pytest.mark.gpu
@needs_addon
def test_addon_end_to_end():
    r = subprocess.run([NODE, "--expose-gc", CHECK], capture_output=True, text=True, timeout=120,
                       cwd=ROOT)
    assert r.returncode == 0, r.stdout + r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["ok"] and out["device"].startswith("gfx950")
    # a readback enqueued before a fill and a free returns the old bytes
    assert out["d2h_async_submission_order"] is True
    # free() followed by GC never returns a block twice
    fg = out["free_then_gc"]
    assert fg["distinct"] and fg["doubleFreeThrows"] and fg["intact"], out
    # bufferPool.getStats()'s names (src/backend/webgpu/buffer.ts:10-15)
    mem = out["mem"]
    for k in ("activeBytes", "pooledBytes", "peakBytes", "allocationCount"):
        assert isinstance(mem[k], (int, float)) and mem[k] >= 0, mem
    assert mem["allocationCount"] >= 1 and mem["allocationRequests"] >= mem["allocationCount"]
