"""CPU checks of the Java FFM adapter (gollek_amd/java/.../GgufHipMatVec.java).

No JDK exists in this image, so the adapter is checked against the C header
as text: every downcall's FunctionDescriptor must have the C declaration's
return and parameter layouts (int32_t -> JAVA_INT, int64_t and size_t ->
JAVA_LONG, pointers -> ADDRESS), every typed wrapper must pass its own
parameters to invokeExact in order with Java types that are exactly those
layouts' carriers (int, long, MemorySegment: no boxing or widening, which
invokeExact rejects at run time), the status constants must equal the
header's, and the reference methods the adapter calls must exist in the
reference sources when those are present.
"""
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
JAVA = REPO / "gollek_amd" / "java" / "tech" / "kayys" / "gollek" / "gguf" / "runtime" / "GgufHipMatVec.java"
HEADER = REPO / "include" / "gollek_hip.h"
REFERENCE = Path("/root/reference")
RT = REFERENCE / "runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf"

CARRIER = {"JAVA_INT": "int", "JAVA_LONG": "long", "ADDRESS": "MemorySegment", "JAVA_FLOAT": "float"}


def c_layout(ctype: str) -> str:
    t = ctype.replace("const", "").strip()
    if "*" in t:
        return "ADDRESS"
    t = t.split()[-1] if t.split() else t
    return {"int32_t": "JAVA_INT", "int64_t": "JAVA_LONG", "size_t": "JAVA_LONG", "float": "JAVA_FLOAT",
            "void": "void"}[t]


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\s*\b(gollek_hip_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        types = []
        for p in plist:
            p = re.sub(r"\b\w+$", "", p).strip() if not p.endswith("*") else p  # drop the name
            types.append(c_layout(p))
        out[name] = (c_layout(ret), types)
    return out


def java_text():
    return JAVA.read_text()


def java_descriptors():
    text = java_text()
    out = {}
    for m in re.finditer(r'downcall\(linker, lookup, "(\w+)",\s*FunctionDescriptor\.(of|ofVoid)\((.*?)\),\s*(true|false)\)',
                         text, flags=re.S):
        name, kind, args = m.group(1), m.group(2), m.group(3)
        layouts = re.findall(r"ValueLayout\.(\w+)", args)
        if kind == "of":
            out[name] = (layouts[0], layouts[1:], m.group(4) == "true")
        else:
            out[name] = ("void", layouts, m.group(4) == "true")
    return out


def test_every_descriptor_matches_the_header():
    hdr = header_functions()
    desc = java_descriptors()
    assert len(desc) >= 8, desc
    for name, (ret, params, _) in desc.items():
        assert name in hdr, f"{name} is not declared in include/gollek_hip.h"
        hret, hparams = hdr[name]
        assert ret == hret, (name, ret, hret)
        assert params == hparams, (name, params, hparams)


def test_heap_array_arguments_use_critical_downcalls():
    # float[] arguments go in as heap segments (MemorySegment.ofArray), which
    # only critical downcalls with heap access accept.
    text = java_text()
    desc = java_descriptors()
    for fn in ("matvecRows", "dotRow", "dequantizeRows", "moeBlock", "moeSharedExpert", "gemmBf16"):
        assert re.search(rf"b\.{fn}\([^;]*MemorySegment\.ofArray", text), fn
    for sym in ("gollek_hip_matvec_rows", "gollek_hip_dot_row", "gollek_hip_dequantize_rows",
                "gollek_hip_moe_block", "gollek_hip_moe_shared_expert", "gollek_hip_gemm_bf16"):
        assert desc[sym][2], sym


WRAPPERS = {  # typed wrapper -> the symbol whose handle it invokes
    "lastStatus": "gollek_hip_last_status",
    "weightUpload": "gollek_hip_weight_upload",
    "weightFree": "gollek_hip_weight_free",
    "weightPrepare": "gollek_hip_weight_prepare",
    "weightUnprepare": "gollek_hip_weight_unprepare",
    "weightCompact": "gollek_hip_weight_compact",
    "matvecRows": "gollek_hip_matvec_rows",
    "dotRow": "gollek_hip_dot_row",
    "dequantizeRows": "gollek_hip_dequantize_rows",
    "moeBlock": "gollek_hip_moe_block",
    "moeSharedExpert": "gollek_hip_moe_shared_expert",
    "gemmBf16": "gollek_hip_gemm_bf16",
}


@pytest.mark.parametrize("wrapper,symbol", sorted(WRAPPERS.items()))
def test_typed_wrappers_call_invoke_exact_with_exact_types(wrapper, symbol):
    text = java_text()
    ret, params, _ = java_descriptors()[symbol]
    m = re.search(rf"\n\s+(int|void|MemorySegment) {wrapper}\(([^)]*)\)\s*\{{(.*?)\n        \}}", text, flags=re.S)
    assert m, wrapper
    jret, jparams, body = m.group(1), m.group(2).strip(), m.group(3)
    decl = [p.strip().rsplit(" ", 1) for p in jparams.split(",")] if jparams else []
    assert [t for t, _ in decl] == [CARRIER[p] for p in params], (wrapper, decl, params)
    assert jret == ("void" if ret == "void" else CARRIER[ret]), (wrapper, jret, ret)
    call = re.search(rf"{wrapper}\.invokeExact\(([^)]*)\)", body)
    assert call, wrapper
    args = [a.strip() for a in call.group(1).split(",")] if call.group(1).strip() else []
    assert args == [n for _, n in decl], (wrapper, args)
    if ret != "void":
        assert re.search(rf"return \({CARRIER[ret]}\) {wrapper}\.invokeExact", body), wrapper


def test_direct_invoke_exact_calls_pass_exact_types():
    # version() and init(...) are invoked in the constructor: an int device
    # (Integer.getInteger unboxed), a MemorySegment and a long length.
    text = java_text()
    assert "Integer.getInteger(\"gollek.hip.device\", 0).intValue()" in text
    assert re.search(r"\(int\) version\.invokeExact\(\)", text)
    assert re.search(r"\(int\) init\.invokeExact\(device, err, \(long\) ERR_LEN\)", text)
    assert re.search(r"private Binding\(Path library, int device\)", text)


def test_status_codes_match_the_header():
    text = java_text()
    hdr = HEADER.read_text()
    for name in ("OK", "ERR_NULL", "ERR_ARG", "ERR_UNSUPPORTED", "ERR_DEVICE", "ERR_NOMEM"):
        h = re.search(rf"#define GOLLEK_HIP_{name} \(?(-?\d+)\)?", hdr)
        j = re.search(rf"static final int {name} = (-?\d+);", text)
        assert h and j and int(h.group(1)) == int(j.group(1)), name


def test_router_scoring_constants_match_the_header():
    text = java_text()
    hdr = HEADER.read_text()
    for name in ("ROUTER_SOFTMAX", "ROUTER_SIGMOID"):
        h = re.search(rf"#define GOLLEK_HIP_{name} (\d+)", hdr)
        j = re.search(rf"static final int {name} = (\d+);", text)
        assert h and j and int(h.group(1)) == int(j.group(1)), name
    # the reference's model-type test, restated in tryMoeLayer
    assert 'mt.contains("qwen") || mt.contains("moe") ? ROUTER_SIGMOID : ROUTER_SOFTMAX' in text


def test_moe_layer_checks_the_lengths_the_library_reads():
    # moe_block and moe_shared_expert take x, logits and the gate row without
    # lengths: the adapter checks them before handing heap arrays over.
    text = java_text()
    body = re.search(r"static boolean tryMoeLayer\((.*?)\n    \}", text, flags=re.S).group(1)
    for cond in ("x.length < (long) tokens * hidden", "logits.length < (long) tokens * (long) nExperts",
                 "sharedGateRow.length < hidden"):
        assert cond in body, cond
    assert body.index("IllegalArgumentException") < body.index("b.moeBlock(")


def test_supported_types_match_the_header():
    text = java_text()
    hdr = HEADER.read_text()
    ids = {int(v) for v in re.findall(r"#define GOLLEK_HIP_Q\w+ (\d+)", hdr)}
    m = re.search(r"static boolean supportsType\(int typeId\) \{\s*return (.*?);", text, flags=re.S)
    assert m and {int(v) for v in re.findall(r"typeId == (\d+)", m.group(1))} == ids


def test_batch_checks_lengths_and_skips_compacted_handles():
    # gemm_bf16 reads m * columns bf16 values and writes m * rows floats: the
    # adapter checks both before handing heap arrays over, creates the handle
    # without a prepared copy, and leaves compacted handles to the mat-vecs.
    text = java_text()
    body = re.search(r"static boolean tryMatVecBatch\((.*?)\n    \}", text, flags=re.S).group(1)
    for cond in ("xRows.length < (long) m * columns", "out.length < (long) m * rows"):
        assert cond in body, cond
    assert "handle(b, model, tensor, rows, columns, rowBytes, false)" in body
    assert "COMPACTED.containsKey(w) && (m > (columns > 4096 ? 2 : 4) || columns > 16384)" in body
    assert body.index("COMPACTED.containsKey(w)") < body.index("b.gemmBf16(")
    assert body.index("IllegalArgumentException") < body.index("b.gemmBf16(")


def _java_bf16(v: float) -> int:
    # GgufHipMatVec.bf16, statement for statement, on 32-bit ints
    import struct
    bits = struct.unpack("<i", struct.pack("<f", v))[0]
    if (bits & 0x7FFFFFFF) > 0x7F800000:
        return (((bits & 0xFFFFFFFF) >> 16) | 0x0040) & 0xFFFF
    return (((bits + 0x7FFF + (((bits & 0xFFFFFFFF) >> 16) & 1)) & 0xFFFFFFFF) >> 16) & 0xFFFF


def test_java_bf16_rounding_is_round_to_nearest_even():
    # The adapter's float -> bf16 rounding, checked against numpy's exact
    # nearest-even rounding through float64 on values around every rounding
    # boundary class: ties to even both ways, carries into the exponent,
    # the largest finite values (rounding to inf), subnormals, signed zeros,
    # infinities and NaNs.
    import numpy as np
    text = java_text()
    assert "return (short) ((bits + 0x7FFF + ((bits >>> 16) & 1)) >>> 16);" in text
    assert "return (short) ((bits >>> 16) | 0x0040);" in text
    rng = np.random.default_rng(7)
    base = rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0x00000000, 0x80000000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F7FFFFF, 0x7F7FFFFF,
                         0x7F7F8000, 0x7F7F7FFF, 0x00008000, 0x00018000, 0x807FFFFF, 0x7F800000, 0xFF800000,
                         0x7FC00000, 0x7F800001, 0xFFFFFFFF], dtype=np.uint32)
    for u in np.concatenate([base, specials, base & 0xFFFF0000 | 0x8000]):
        f = float(np.uint32(u).view(np.float32))
        got = _java_bf16(f)
        if np.isnan(f):
            assert (got & 0x7F80) == 0x7F80 and (got & 0x7F) != 0, hex(int(u))
            continue
        if np.isinf(f):
            assert got == int(u) >> 16, hex(int(u))
            continue
        # exact nearest-even between the two bf16 neighbours of the same sign
        # (a neighbour past the largest finite bf16 counts as +-2^128)
        lo = int(u) >> 16
        hi = lo + 1
        v_lo = float(np.uint32(lo << 16).view(np.float32))
        v_hi = (float(np.uint32(hi << 16).view(np.float32)) if (hi & 0x7FFF) != 0x7F80
                else float(np.copysign(2.0 ** 128, f)))
        d_lo, d_hi = abs(f - v_lo), abs(v_hi - f)
        want = lo if d_lo < d_hi or (d_lo == d_hi and lo % 2 == 0) else hi
        assert got == (want & 0xFFFF), (hex(int(u)), hex(got), hex(want))


@pytest.mark.skipif(not RT.exists(), reason="reference sources not present")
def test_reference_methods_the_adapter_calls_exist():
    # GgufTensorData.tensorData(GGUFModel, GGUFTensorInfo) -> MemorySegment,
    # GGUFTensorInfo.typeId(), and the hooks' host methods.
    td = (RT / "runtime" / "GgufTensorData.java").read_text()
    assert re.search(r"static MemorySegment tensorData\(GGUFModel model, GGUFTensorInfo tensor\)", td)
    info = (RT / "loader" / "GGUFTensorInfo.java").read_text()
    assert re.search(r"record GGUFTensorInfo\(", info) and "int typeId" in info
    model = (RT / "loader" / "GGUFModel.java").read_text()
    assert "public final class GGUFModel" in model
    mv = (RT / "runtime" / "GgufMatVec.java").read_text()
    assert "static void rows(" in mv and "layout.rowBytes()" in mv and "package tech.kayys.gollek.gguf.runtime;" in mv
    ops = (RT / "runtime" / "GgufTensorOps.java").read_text()
    assert "public static float dotRow(GGUFModel model, GGUFTensorInfo tensor, long row, float[] vector)" in ops
    assert "public static void dequantizeRow(GGUFModel model, GGUFTensorInfo tensor, long row, float[] dst)" in ops
    assert "clearPreparedMatrixCaches" in ops
    java = java_text()
    assert "package tech.kayys.gollek.gguf.runtime;" in java
    assert "GgufTensorData.tensorData(model, tensor)" in java
    # tryMoeLayer: GGUFTensorInfo.shape() and sizeInBytes(), and the
    # MoeForwardPass lines it replaces
    assert "long[] shape" in info and "long sizeInBytes" in info
    moe = (REFERENCE / "runner/safetensor/gollek-safetensor-engine/src/main/java/tech/kayys/gollek/"
           "safetensor/engine/generation/moe/MoeForwardPass.java").read_text()
    assert 'modelType.contains("qwen") || modelType.contains("moe")' in moe
    assert "runSharedExpert(" in moe and "resolveSharedExpertGate(" in moe
