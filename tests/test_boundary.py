"""The drop-in boundary on the CPU: the C-ABI library loads and exports every declared symbol, the
Backend and Compiler seams answer as the reference's traits do, the lifts build the reference's
kernels (and decline where it declines), and lower_kernel recognises exactly those kernels."""
from __future__ import annotations

import copy
import ctypes as C
import json
import re
from pathlib import Path

import pytest

import unpopped_amd as u
from unpopped_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> list[str]:
    text = (ROOT / "include" / "unpopped_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(unp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = C.CDLL(str(_lib.LIB_PATH))
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_backend_identity():
    b = u.HipBackend()
    assert b.name() == "hip"
    assert b.provider() == "unpopped-hip"
    assert b.total_integer_ops() is True


def test_supports_dtype_is_target_conditional():
    b = u.HipBackend()
    for dt in ("F32", "F64", "I32", "I64", "Bf16", "F16", "U4", "I4", "U32"):
        assert b.supports_dtype(dt, "rocm:gfx950") == "Supported", dt
    assert b.supports_dtype("F32", "cuda:sm89") == "Unsupported"
    assert b.supports_dtype("F32", "rocm:gfx942") == "Unsupported"
    assert b.supports_dtype("Fp8E4M3FN", "rocm:gfx950") == "Unsupported"
    for bad in ("rocm", "rocm:", ":gfx950", "rocm:gfx|950", "rocm:gfx 950", "a:b:c"):
        assert b.supports_dtype("F32", bad) == "Unsupported", bad


def test_compiler_produces_a_gfx950_code_object():
    cc = u.HipCompiler()
    assert cc.artifact_kind() == "HipCodeObject"
    src = 'extern "C" __global__ void k(float* x) { x[threadIdx.x] *= 2.0f; }'
    co = cc.compile(src, "k")
    assert co[:4] == b"\x7fELF"
    assert b"gfx950" in co
    with pytest.raises(_lib.UnpError) as e:
        cc.compile("this is not HIP", "k")
    assert e.value.kind == "CompileError" and "error" in e.value.detail


def test_revision_hash_is_fnv1a_over_the_source():
    g = u.HipBackend().lower_kernel(u.lift_scan("s", "I32", 1, "Sum", launch=(64, 1)))
    h = 0xCBF29CE484222325
    for byte in g.source.encode():
        h = ((h ^ byte) * 0x100000001B3) & ((1 << 64) - 1)
    assert g.revision_hash() == h


# ---------------------------------------------------------------------------------------
# The lifts
# ---------------------------------------------------------------------------------------

def stmts(kernel):
    """Every statement of a kernel body, depth first."""
    out = []

    def walk(block):
        for s in block:
            out.append(s)
            (name, body), = s.items() if isinstance(s, dict) else (("", None),)
            if isinstance(body, dict):
                for key in ("then", "els", "body"):
                    if key in body:
                        walk(body[key])

    walk(kernel["body"])
    return out


def test_launched_reduction_has_the_reference_shape():
    """kernel_lift/block_reduce.rs: Shared `partial` (f64 for a float) and `partial_have` for
    Max/Min, log2(block) tree rounds each followed by a barrier, launch [block,1,1] x [grid,1,1]."""
    k = u.lift_reduction("r", "F32", 2, "Max", launch=(128, 7))
    assert [a["name"] for a in k["allocs"]] == ["partial", "partial_have"]
    assert k["allocs"][0]["elem"] == "F64" and k["allocs"][0]["extent"] == {"Static": 128}
    assert k["launch"]["block"] == [128, 1, 1] and k["launch"]["grid"] == [7, 1, 1]
    barriers = [s for s in stmts(k) if "Barrier" in s]
    assert len(barriers) == 1 + 7  # after the publish, then one per tree round (128 = 2^7)
    assert [p["name"] for p in k["params"]] == ["in0", "out", "n0", "n1"]
    s = u.lift_reduction("r", "I64", 2, "Sum", launch=(64, 1))
    assert [a["name"] for a in s["allocs"]] == ["partial"] and s["allocs"][0]["elem"] == "I64"
    serial = u.lift_reduction("r", "F32", 2, "Sum")
    assert serial["launch"] is None and serial["allocs"] == []


def test_launched_scan_has_the_reference_shape():
    k = u.lift_scan("s", "F32", 1, "Sum", launch=(16, 1))
    first = k["body"][0]
    assert first == {"Let": {"local": 7, "init": {"ConstInt": [0, "I32"]}}}  # chunk = 0 (scan_launched.rs:190)
    assert "While" in k["body"][1]
    barriers = [s for s in stmts(k) if "Barrier" in s]
    assert len(barriers) == 1 + 2 * 4 + 1  # publish, 2 per Kogge-Stone round (16 = 2^4), end of row


def test_lift_declines_match_the_reference():
    def decline(fn, *a, **kw):
        with pytest.raises(_lib.UnpError) as e:
            fn(*a, **kw)
        assert e.value.kind == "LiftDecline"
        return e.value.detail

    assert decline(u.lift_reduction, "r", "F32", 1, "Sum", launch=(96, 1)) == "BadLaunch"  # not a power of two
    assert decline(u.lift_reduction, "r", "F32", 1, "Sum", launch=(64, 0)) == "BadLaunch"
    assert "float Prod" in decline(u.lift_reduction, "r", "F32", 1, "Prod", launch=(64, 1))
    assert "integer Mean" in decline(u.lift_reduction, "r", "I32", 1, "Mean")
    assert decline(u.lift_reduction, "r", "F32", 9, "Sum") == "BadRank"
    assert "outside F32" in decline(u.lift_reduction, "r", "Bf16", 1, "Sum")
    assert "non-innermost" in decline(u.lift_scan, "s", "F32", 2, "Sum", axis=0, launch=(64, 1))
    assert "Mean scan" in decline(u.lift_scan, "s", "F32", 1, "Mean", launch=(64, 1))
    assert "non-integer" in decline(u.lift_gather, "g", "F32", 2, "F32")
    assert decline(u.lift_gather, "g", "F32", 2, launch=(64, 0)) == "BadLaunch"
    # the serial lifts accept what the launched ones decline
    u.lift_reduction("r", "F32", 1, "Prod")
    u.lift_scan("s", "F32", 2, "Sum", axis=0)
    u.lift_scan("s", "F64", 1, "Mean")


# ---------------------------------------------------------------------------------------
# lower_kernel
# ---------------------------------------------------------------------------------------

CASES = [
    (lambda: u.lift_reduction("r", "F32", 2, "Sum", launch=(256, 64)), "lift_reduction_opdef_launched", "unp_rowreduce_sum_f32"),
    (lambda: u.lift_reduction("r", "F32", 1, "Sum", launch=(256, 1)), "lift_reduction_opdef_launched", "unp_reduce_all_sum_f32"),
    (lambda: u.lift_reduction("r", "F64", 3, "Mean", axes=(1, 2), keepdim=True), "lift_reduction_opdef", "unp_rowreduce_mean_f64"),
    (lambda: u.lift_reduction("r", "I64", 2, "Prod", launch=(32, 3)), "lift_reduction_opdef_launched", "unp_rowreduce_prod_i64"),
    (lambda: u.lift_reduction("r", "I32", 2, "Min", axes=(0, 1)), "lift_reduction_opdef", "unp_reduce_all_min_i32"),
    (lambda: u.lift_scan("s", "I32", 1, "Sum", launch=(256, 1)), "lift_scan_opdef_launched", "unp_scan_incl_sum_i32"),
    (lambda: u.lift_scan("s", "F32", 3, "Max", exclusive=True, reverse=True), "lift_scan_opdef", "unp_scan_fix_excl_rev_max_f32"),
    (lambda: u.lift_scan("s", "I64", 2, "Prod", exclusive=True, launch=(64, 8)), "lift_scan_opdef_launched", "unp_scan_excl_prod_i64"),
    (lambda: u.lift_gather("e", "Bf16", 2, "I32", launch=(256, 4096)), "lift_gather_opdef_launched", "unp_gather_rows_bf16_by_i32_ZeroFill"),
    (lambda: u.lift_gather("g", "U8", 3, "I64", oob="Skip"), "lift_gather_opdef", "unp_gather_rows_u8_by_i64_Skip"),
    (lambda: u.lift_gather("g", "F64", 2, "U32", oob="Clamp", launch=(64, 2)), "lift_gather_opdef_launched", "unp_gather_rows_f64_by_u32_Clamp"),
    (lambda: u.kernel_row_reduce2("p", "F32", "Sum", "Max"), "row_reduce2", "unp_rowreduce_sum_max_f32"),
    (lambda: u.kernel_dequant4("d", "I4", "U4", 128, launch=(64, 64)), "dequant4", "unp_dequant_i4_zu4_g128_bf16"),
    (lambda: u.kernel_dequant_gemm("m", "I4", "I32", 128), "dequant_gemm", "unp_dequant_gemm_i4_g128_i32_i32"),
    (lambda: u.kernel_dequant_gemm("m", "U4", "I8", 64, launch=(256, 8)), "dequant_gemm", "unp_dequant_gemm_u4_g64_i8_i32"),
]


@pytest.mark.parametrize("make,lift,name", CASES)
def test_lower_kernel_recognises_the_lifts(make, lift, name):
    k = make()
    g = u.HipBackend().lower_kernel(k)
    assert g.interface["lift"] == lift
    assert g.name == name
    assert g.interface["kernel"] == k["name"]
    assert g.interface["declared_launch"] == k["launch"]
    assert g.interface["kernel_params"] == k["params"]
    assert 'extern "C" __global__' in g.source and "rocm:gfx950" in g.source
    assert g.interface["fidelity_notes"]


def test_lower_kernel_accepts_serde_defaults_left_out():
    k = u.lift_reduction("r", "F32", 2, "Sum", launch=(256, 64))
    slim = copy.deepcopy(k)
    for key in ("allocs", "result", "results"):
        slim.pop(key)
    slim["allocs"] = k["allocs"]  # a launched reduction needs its allocations
    for key in ("cluster", "devices", "grid_dims"):
        slim["launch"].pop(key)

    def drop_unroll(x):
        if isinstance(x, dict):
            if "For" in x and isinstance(x["For"], dict):
                x["For"].pop("unroll", None)
            for v in x.values():
                drop_unroll(v)
        elif isinstance(x, list):
            for v in x:
                drop_unroll(v)

    drop_unroll(slim)
    assert u.HipBackend().lower_kernel(json.dumps(slim)).interface["lift"] == "lift_reduction_opdef_launched"


def mutated(k, path, value):
    k = copy.deepcopy(k)
    node = k
    for p in path[:-1]:
        node = node[p]
    node[path[-1]] = value
    return k


def test_lower_kernel_refuses_anything_else():
    b = u.HipBackend()

    def refused(k, kind="UnsupportedKernel"):
        with pytest.raises(_lib.UnpError) as e:
            b.lower_kernel(k)
        assert e.value.kind == kind, e.value.detail
        return e.value.detail

    k = u.lift_reduction("r", "F32", 2, "Sum", launch=(256, 64))
    # a different fold (Sub instead of Add in the accumulate) is not a lift's kernel
    text = json.dumps(k).replace('{"Assign": {"local": 5, "value": {"Add":', '{"Assign": {"local": 5, "value": {"Sub":', 1)
    assert text != json.dumps(k)
    refused(text)
    # an extra statement
    extra = copy.deepcopy(k)
    extra["body"].append({"Barrier": {"scope": "Block", "kind": "Full"}})
    refused(extra)
    # a different launch geometry inside the tree than declared
    refused(mutated(k, ["launch", "block"], [128, 1, 1]))
    # not JSON, not a KernelFn
    refused("{not json", "ParseError")
    refused(json.dumps([1, 2, 3]), "ParseError")
    # a gather along axis 1 (index_select) is recognised and lowered to the batched row gather
    assert b.lower_kernel(u.lift_gather("g", "F32", 2, axis=1)).interface["axis"] == 1
    # a float Prod: the serial lift is lowered to the entry that multiplies in the serial order; the
    # launched lift declines it (block_reduce.rs:97-133)
    assert b.lower_kernel(u.lift_reduction("r", "F32", 2, "Prod")).name.startswith("unp_reduce_serial_prod_f32")
    with pytest.raises(_lib.UnpError) as e:
        u.lift_reduction("r", "F32", 2, "Prod", launch=(256, 64))
    assert e.value.kind == "LiftDecline" and "float Prod" in e.value.detail
    # a scan along a non-innermost axis: the serial lift, lowered to the serial-order scan; the
    # launched lift declines it (kernel_lift.rs:689-695)
    g = b.lower_kernel(u.lift_scan("s", "F32", 2, "Sum", axis=0))
    assert g.interface["schedule"] == "serial" and g.interface["axis"] == 0
    with pytest.raises(_lib.UnpError) as e:
        u.lift_scan("s", "F32", 2, "Sum", axis=0, launch=(256, 64))
    assert "non-innermost" in e.value.detail
    # a pre-map body (x * x) is the lift of OpDef::reduction with that body: recognised, and
    # spelled into the kernel (kernel_lift.rs:919-941)
    sq = json.dumps(u.lift_reduction("r", "F64", 1, "Sum")).replace(
        '{"Let": {"local": 5, "init": {"Local": 2}}}',
        '{"Let": {"local": 5, "init": {"Mul": [{"Local": 2}, {"Local": 2}]}}}')
    assert '"Mul"' in sq
    g = b.lower_kernel(sq)
    assert g.interface["body"] == "(x[0] * x[0])" and g.interface["post"] is None
    # a body that reads a local other than a loaded input (here an extent) is no lift's kernel
    ext = json.dumps(u.lift_reduction("r", "F64", 1, "Sum")).replace(
        '{"Let": {"local": 5, "init": {"Local": 2}}}', '{"Let": {"local": 5, "init": {"Local": 0}}}')
    refused(ext)


def test_lower_form_declines_unsupported_forms():
    b = u.HipBackend()
    for form, kind in [
        (dict(kind="reduction", dtype="F32", op="And", rank=1, reduced_from=0), "UnsupportedKernel"),
        (dict(kind="reduction", dtype="I32", op="Mean", rank=1, reduced_from=0), "UnsupportedKernel"),
        (dict(kind="scan", dtype="I32", op="Mean"), "UnsupportedKernel"),
        (dict(kind="gather", dtype="U4", rank=2), "UnsupportedDtype"),
        (dict(kind="dequant4", out_kind="F32"), "UnsupportedDtype"),
        (dict(kind="dequant4", group=0), "UnsupportedKernel"),
        (dict(kind="dequant_gemm", q_kind="I8", dtype="I32"), "UnsupportedDtype"),
        (dict(kind="dequant_gemm", q_kind="U4", dtype="F32"), "UnsupportedDtype"),
        (dict(kind="reduction", dtype="F32", rank=9), "LiftDecline"),
    ]:
        with pytest.raises(_lib.UnpError) as e:
            b.lower_form(**form)
        assert e.value.kind == kind, (form, e.value.kind, e.value.detail)


def test_every_lowered_source_compiles_for_gfx950():
    """The Compiler seam on each form's emitted source (hipRTC needs no GPU)."""
    b, cc = u.HipBackend(), u.HipCompiler()
    seen = set()
    for make, _, _ in CASES:
        g = b.lower_kernel(make())
        if g.name in seen:
            continue
        seen.add(g.name)
        co = cc.compile(g.source, g.name)
        for e in g.interface["entries"]:
            assert e["symbol"].encode() in co


# ---------------------------------------------------------------------------------------
# Access::RowReduce (kernel_lift/row_reduce.rs, row_reduce_launched.rs)
# ---------------------------------------------------------------------------------------

from unpopped_amd import expr as X  # noqa: E402

ROW_REDUCTIONS = {"softmax": X.softmax(), "centred_quotient": X.centred_quotient(), "rms_norm": X.rms_norm(),
                  "identity_sum": ([(X.input(0), "Sum")], X.reduced(0))}


@pytest.mark.parametrize("which", sorted(ROW_REDUCTIONS))
@pytest.mark.parametrize("dtype", ["F32", "F64"])
@pytest.mark.parametrize("launch", [None, (256, 64), (1, 3)])
def test_row_reduce_lifts_round_trip(which, dtype, launch):
    stages, epi = ROW_REDUCTIONS[which]
    k = u.lift_row_reduce(which, dtype, 2, stages, epi, launch=launch)
    g = u.HipBackend().lower_kernel(k)
    assert g.interface["lift"] == ("lift_row_reduce_opdef_launched" if launch else "lift_row_reduce_opdef")
    assert [s["op"] for s in g.interface["stages"]] == [op for _, op in stages]
    assert g.name.startswith(f"unp_row_reduce_{dtype.lower()}_s{len(stages)}_")
    assert [e["symbol"].rsplit("_", 1)[1] for e in g.interface["entries"]] == ["c4", "c", "v", "s"]
    # softmax's exp(x - max) is the Sum stage's pre value and recurs in the epilogue: the
    # register-resident entries keep it instead of evaluating exp twice.  Cheap or absent
    # subexpressions are not held.
    assert g.interface["epilogue_reuses_stage"] == (1 if which == "softmax" else -1)
    if which == "softmax":
        # An f32 output multiplies the kept value by the row's reciprocal; an f64 output divides.
        flat = g.source.replace("(", "").replace(")", "")
        assert "epi_c" in g.source and ("c * 1.0 / r[1]" if dtype == "F32" else "c / r[1]") in flat
        assert ("reciprocal" in g.interface["fidelity_notes"][-1]) == (dtype == "F32")


def test_row_reduce_launched_shape():
    """row_reduce_launched.rs: per stage a strided fold, the block tree, thread 0's rounding into
    Shared slot s and a broadcast load; allocations partial (F64), partial_have, stage_result."""
    stages, epi = X.softmax()
    k = u.lift_row_reduce("sm", "F32", 2, stages, epi, launch=(16, 2))
    assert [a["name"] for a in k["allocs"]] == ["partial", "partial_have", "stage_result"]
    assert [a["elem"] for a in k["allocs"]] == ["F64", "I32", "F32"]
    assert k["allocs"][2]["extent"] == {"Static": 2}
    barriers = [s for s in stmts(k) if "Barrier" in s]
    assert len(barriers) == 2 * (1 + 4 + 1)  # per stage: publish, log2(16) rounds, the broadcast
    # serial: locals 2r + (S+1)n + 4S; launched: one more (the partner's have)
    ks = u.lift_row_reduce("sm", "F32", 2, stages, epi)
    assert len(ks["locals"]) == 4 + 3 + 8 and len(k["locals"]) == 4 + 3 + 8 + 1


def test_row_reduce_declines():
    def decline(*a, **kw):
        with pytest.raises(_lib.UnpError) as e:
            u.lift_row_reduce(*a, **kw)
        assert e.value.kind == "LiftDecline"
        return e.value.detail

    sm = X.softmax()
    assert "Prod stage" in decline("p", "F32", 2, [(X.input(0), "Prod")], X.reduced(0), launch=(64, 1))
    assert "leading axis" in decline("p", "F32", 1, *sm, launch=(64, 1))
    assert decline("p", "F32", 2, *sm, launch=(96, 1)) == "BadLaunch"
    assert "non-float" in decline("p", "F16", 2, *sm)
    assert "empty stage" in decline("p", "F32", 2, [], X.input(0))
    assert "later stage" in decline("p", "F32", 2, [(X.reduced(0), "Sum")], X.input(0))
    assert "Param" in decline("p", "F32", 2, [({"Param": 0}, "Sum")], X.reduced(0))
    assert decline("p", "F32", 9, *sm) == "BadRank"
    # the serial lift takes a Prod stage
    u.lift_row_reduce("p", "F32", 2, [(X.input(0), "Prod")], X.reduced(0))


def test_row_reduce_refusals_are_typed():
    b = u.HipBackend()
    # a Prod stage lifts (serially) but this backend declares no order-independent kernel for it
    k = u.lift_row_reduce("p", "F32", 2, [(X.input(0), "Prod")], X.reduced(0))
    with pytest.raises(_lib.UnpError) as e:
        b.lower_kernel(k)
    assert e.value.kind == "UnsupportedKernel" and "Prod" in e.value.detail
    # an op this backend has no spelling for is an UnsupportedOp
    k = u.lift_row_reduce("g", "F32", 2, [(X.input(0).unary("Lgamma"), "Sum")], X.reduced(0))
    with pytest.raises(_lib.UnpError) as e:
        b.lower_kernel(k)
    assert e.value.kind == "UnsupportedOp" and "Lgamma" in e.value.detail
    # a perturbed kernel is not a row reduction: the epilogue stored into the wrong buffer
    k = u.lift_row_reduce("sm", "F32", 2, *X.softmax(), launch=(64, 4))
    text = json.dumps(k).replace('{"Barrier": {"scope": "Block", "kind": "Full"}}', '{"Barrier": {"scope": "Block", "kind": "Full"}}, {"Barrier": {"scope": "Block", "kind": "Full"}}', 1)
    with pytest.raises(_lib.UnpError) as e:
        b.lower_kernel(text)
    assert e.value.kind == "UnsupportedKernel"


def test_row_reduce_two_inputs_and_rank_three():
    b = u.HipBackend()
    k = u.lift_row_reduce("two", "F64", 3, [(X.input(0) * X.input(1), "Sum")],
                          X.input(0) * X.reduced(0) + X.input(1), n_inputs=2, launch=(128, 8))
    g = b.lower_kernel(k)
    assert g.interface["inputs"] == 2 and g.interface["rank"] == 3
    assert g.interface["epilogue"] == "((x[0] * r[0]) + x[1])"
    u.HipCompiler().compile(g.source, g.name)


def test_dequant_gemm_entries_follow_the_group():
    """The decode entries (1, 2 and 4 column tiles for I8 activations, one for I32) and their prep
    exist when the group holds 1..4 whole 128-value steps (1..2 for I32), the streaming entry and
    its prep when it holds whole 64-value chunks, the LDS-transpose MFMA entry when it holds whole
    32-deep steps, the serial entry always; each staged chunk divides the group."""
    b = u.HipBackend()
    for w_kind, x_kind, group, chunk, stream, dec in (
            ("I4", "I32", 128, 128, 64, 2), ("I4", "I32", 256, 128, 64, 2), ("U4", "I32", 512, 128, 64, 0),
            ("U4", "I8", 128, 128, 128, 2), ("U4", "I8", 512, 512, 128, 4), ("U4", "I8", 384, 384, 128, 3),
            ("U4", "I8", 1024, 512, 128, 0), ("U4", "I8", 64, 64, 64, 0), ("U4", "I8", 96, 96, 0, 0),
            ("I4", "I32", 7, 0, 0, 0), ("U4", "I8", 48, 0, 0, 0)):
        g = b.lower_kernel(u.kernel_dequant_gemm("m", w_kind, x_kind, group))
        assert g.interface["form"] == "dequant_gemm" and g.interface["group"] == group
        assert g.interface["chunk"] == chunk and (chunk == 0 or group % chunk == 0)
        assert g.interface["stream_chunk"] == stream and (stream == 0 or group % stream == 0)
        # The decode entry keeps a whole number of groups in flight.
        assert g.interface["decode_steps"] == dec and (dec == 0 or dec % (group // 128) == 0)
        syms = [e["symbol"].rsplit("_", 1)[1] for e in g.interface["entries"]]
        decs = (["dec1x", "dec2", "dec4"] if x_kind == "I8" else ["dec1"]) if dec else []
        want = (decs + (["stream"] if stream else []) + (["mfma"] if chunk else []) + ["any"]
                + (["prep"] if stream else []) + (["prep16"] if dec else []))
        assert syms == want


def test_dequant_gemm_refuses_other_element_types():
    with pytest.raises(_lib.UnpError):
        u.kernel_dequant_gemm("m", "U4", "F32", 128)
    k = u.kernel_dequant_gemm("m", "U4", "I32", 128)
    k["params"][3]["kind"]["Buffer"]["elem"] = "I16"
    with pytest.raises(_lib.UnpError):
        u.HipBackend().lower_kernel(k)


def test_bit_and_nan_ignoring_folds_lift_only_sequentially():
    """And/Or/Xor (integers) and MaxNum/MinNum lift as sequential reductions only
    (kernel_lift.rs:763-800, block_reduce.rs:97-133): the serial lift is recognised and lowered, the
    launched lift, a scan and a float bit fold are typed declines."""
    be = u.HipBackend()
    for dt, op in (("F32", "MaxNum"), ("F64", "MinNum"), ("I32", "And"), ("I64", "Or"), ("I32", "Xor")):
        for axes in ((1,), (0,), (0, 1)):
            g = be.lower_kernel(u.lift_reduction("r", dt, 2, op, axes=axes))
            assert op.lower() in g.name, (dt, op, g.name)
        with pytest.raises(_lib.UnpError) as e:
            u.lift_reduction("r", dt, 2, op, launch=(256, 64))
        assert e.value.kind == "LiftDecline" and "sequential lift only" in e.value.detail
        with pytest.raises(_lib.UnpError):
            u.lift_scan("s", dt, 1, op)
    for op in ("And", "Or", "Xor"):
        with pytest.raises(_lib.UnpError) as e:
            u.lift_reduction("r", "F32", 2, op)
        assert "bit reduction at a float dtype" in e.value.detail


def test_mean_and_float_prod_scans_lift_only_sequentially():
    """A Mean scan and a float Prod scan have serial lifts only (kernel_lift/scan_launched.rs:66-75):
    the serial lift is lowered (Mean on the look-back scan with the division at the store, a float
    Prod in the serial order), the launched lift declines, and an integer Mean declines."""
    b = u.HipBackend()
    assert b.lower_kernel(u.lift_scan("s", "F32", 1, "Mean")).name.startswith("unp_scan_fix_incl_mean_f32")
    assert b.lower_kernel(u.lift_scan("s", "F64", 1, "Prod", exclusive=True)).name.startswith("unp_scan_seq_excl_prod")
    for op in ("Mean", "Prod"):
        with pytest.raises(_lib.UnpError) as e:
            u.lift_scan("s", "F32", 1, op, launch=(256, 64))
        assert e.value.kind == "LiftDecline"
    with pytest.raises(_lib.UnpError) as e:
        u.lift_scan("s", "I32", 1, "Mean")
    assert "integer Mean" in e.value.detail


# ---------------------------------------------------------------------------------------
# Recognition up to a consistent renumbering of locals and any key order
# ---------------------------------------------------------------------------------------

def renumber_locals(k: dict, perm: list[int]) -> dict:
    """``k`` with local i renamed perm[i] everywhere it is referenced (the ScalarExpr leaf Local(n), the
    ``local`` of Let/Load/Assign/For and of a Scalar parameter) and its locals list permuted to match."""
    k = copy.deepcopy(k)

    def walk(x):
        if isinstance(x, dict):
            if len(x) == 1 and isinstance(x.get("Local"), int):
                x["Local"] = perm[x["Local"]]
                return
            for key, v in x.items():
                if key == "local" and isinstance(v, int):
                    x[key] = perm[v]
                else:
                    walk(v)
        elif isinstance(x, list):
            for v in x:
                walk(v)

    walk(k["params"])
    walk(k["body"])
    locs = [None] * len(k["locals"])
    for old, new in enumerate(perm):
        locs[new] = k["locals"][old]
    k["locals"] = locs
    return k


def shuffle_keys(x, rng):
    """The same JSON value with every object's keys in a random order."""
    if isinstance(x, dict):
        items = list(x.items())
        rng.shuffle(items)
        return {key: shuffle_keys(v, rng) for key, v in items}
    if isinstance(x, list):
        return [shuffle_keys(v, rng) for v in x]
    return x


def _renumber_cases():
    from unpopped_amd import expr as X

    x0, x1, r0 = X.input(0), X.input(1), X.reduced(0)
    stages, epi = X.softmax()
    out = [make for make, _, _ in CASES]
    out += [
        lambda: u.lift_reduction("xr", "F32", 2, "Sum", axes=(1,), launch=(256, 64), n_inputs=2, body=x0 * x1,
                                 post=r0.sqrt()),
        lambda: u.lift_reduction("xr", "F64", 3, "Max", axes=(0, 2), n_inputs=2, body=x0 - x1),
        lambda: u.lift_reduction("mn", "F32", 2, "MaxNum", axes=(0,)),
        lambda: u.lift_scan("s", "F64", 3, "Mean", axis=1, exclusive=True),
        lambda: u.lift_gather("g", "I32", 3, "U32", axis=2, oob="Skip", launch=(64, 3)),
        lambda: u.lift_row_reduce("softmax", "F32", 2, stages, epi, launch=(256, 64)),
        lambda: u.lift_row_reduce("softmax", "F64", 3, stages, epi),
        lambda: u.lift_gather("gx", "F32", 2, "I32", oob="ZeroFill", n_inputs=3, data=2, index=0,
                              body=X.input(2) * X.input(1) + 0.5, launch=(64, 4)),
        lambda: u.lift_gather("gx", "I64", 3, "U32", axis=1, oob="Skip", n_inputs=3, data=0, index=2,
                              body=X.input(0)),
        lambda: u.lift_scan("sx", "F32", 2, "Sum", n_inputs=2, pre=x0 * x1, post=r0 - x0, launch=(256, 64)),
        lambda: u.lift_scan("sx", "F64", 3, "Mean", axis=0, exclusive=True, reverse=True, n_inputs=2,
                            pre=x0 + x1, post=r0.sqrt()),
        lambda: u.lift_scan("sx", "F32", 1, "Max", n_inputs=1, pre=x0 * x0),
    ]
    return out


@pytest.mark.parametrize("i", range(len(_renumber_cases())))
def test_lower_kernel_tolerates_renumbered_locals_and_key_order(i):
    """A kernel equal to a lift up to a consistent renumbering of its locals, with its object keys in any
    order, is recognised as that lift and lowers to the same HIP source."""
    import random

    k = _renumber_cases()[i]()
    b = u.HipBackend()
    want = b.lower_kernel(k)
    rng = random.Random(1000 + i)
    for _ in range(3):
        perm = list(range(len(k["locals"])))
        rng.shuffle(perm)
        moved = shuffle_keys(renumber_locals(k, perm), rng)
        assert moved != k
        g = b.lower_kernel(json.dumps(moved))
        assert g.name == want.name and g.source == want.source
        assert g.interface["lift"] == want.interface["lift"]
    # the reverse numbering too (every id moves)
    g = b.lower_kernel(renumber_locals(k, list(range(len(k["locals"])))[::-1]))
    assert g.source == want.source


def test_inconsistent_renumbering_is_refused():
    """Renaming one reference of a local (not all of them) changes the kernel: refused."""
    k = u.lift_reduction("r", "F32", 2, "Sum", launch=(256, 64))
    text = json.dumps(k)
    # the accumulator (local 5) renamed in its Let only: its folds still read local 5
    bad = text.replace('{"Let": {"local": 5, "init"', '{"Let": {"local": 7, "init"', 1)
    assert bad != text
    with pytest.raises(_lib.UnpError) as e:
        u.HipBackend().lower_kernel(bad)
    assert e.value.kind == "UnsupportedKernel"
    # a permuted locals list without renaming the references: the declared types no longer line up
    k2 = copy.deepcopy(k)
    k2["locals"] = k2["locals"][::-1]
    with pytest.raises(_lib.UnpError) as e:
        u.HipBackend().lower_kernel(k2)
    assert e.value.kind == "UnsupportedKernel"


# ---------------------------------------------------------------------------------------
# The lifts' parameter names, local layout and statement skeletons, pinned to the reference
# ---------------------------------------------------------------------------------------

def _place(p):
    (kind, b), = p.items()
    return ("buf", b["buffer"]) if kind == "Logical" else ("shared", b["alloc"])


def skeleton(block):
    """Statement kinds with the locals and places they name, nested as in the body."""
    out = []
    for st in block:
        (kind, b), = st.items()
        if kind == "For":
            out.append(("For", b["local"], skeleton(b["body"])))
        elif kind == "Let":
            out.append(("Let", b["local"]))
        elif kind == "Load":
            out.append(("Load", b["local"], _place(b["place"])))
        elif kind == "Assign":
            out.append(("Assign", b["local"]))
        elif kind == "Store":
            out.append(("Store", _place(b["place"])))
        elif kind == "If":
            out.append(("If", skeleton(b["then"]), skeleton(b["els"])))
        elif kind == "While":
            out.append(("While", skeleton(b["body"])))
        else:
            out.append((kind,))
    return out


def _sig(k):
    params = []
    for p in k["params"]:
        (kind, b), = p["kind"].items()
        params.append((p["name"], kind, b.get("rank") if kind == "Buffer" else b["local"]))
    return params, [loc["elem"] for loc in k["locals"]]


# extremum_step (kernel_lift.rs:1097-1129) with nan_arm (:1134-1160) for a float Max/Min:
#   if have { if v != v { acc = v } else { if better(v, acc) { acc = v } } } else { acc = v }; have = 1
def _float_extremum(acc, have):
    return [("If", [("If", [("Assign", acc)], [("If", [("Assign", acc)], [])])], [("Assign", acc)]),
            ("Assign", have)]


# ... and for MaxNum/MinNum: if acc != acc { acc = v } else { if v == v { if better { acc = v } } }
def _num_extremum(acc, have):
    return [("If", [("If", [("Assign", acc)], [("If", [("If", [("Assign", acc)], [])], [])])], [("Assign", acc)]),
            ("Assign", have)]


def test_serial_reduction_skeleton_follows_kernel_lift():
    """lift_reduction_opdef (kernel_lift.rs:447-484): locals extents 0..r, counters r..2r, loaded inputs
    2r..2r+n, then acc, have, val (:440-442, signature :1006-1024); per kept row `acc`/`have` Lets, the
    reduced loops around the loads, `val` and the fold step (reduce_loop :919-941), one Store."""
    k = u.lift_reduction("r", "F32", 2, "Max", axes=(1,))
    params, locals_ = _sig(k)
    assert params == [("in0", "Buffer", 2), ("out", "Buffer", 1), ("n0", "Scalar", 0), ("n1", "Scalar", 1)]
    assert locals_ == ["I32"] * 4 + ["F32", "F64", "I32", "F64"]
    assert skeleton(k["body"]) == [
        ("For", 2, [("Let", 5), ("Let", 6),
                    ("For", 3, [("Load", 4, ("buf", 0)), ("Let", 7), *_float_extremum(5, 6)]),
                    ("Store", ("buf", 1))])]
    # Sum: one Assign acc = acc + val (fold_step :1049-1060); the reduced axis 0 nests inside kept axis 1
    s = u.lift_reduction("r", "I64", 2, "Sum", axes=(0,))
    assert skeleton(s["body"]) == [
        ("For", 3, [("Let", 5), ("Let", 6), ("For", 2, [("Load", 4, ("buf", 0)), ("Let", 7), ("Assign", 5)]),
                    ("Store", ("buf", 1))])]
    assert s["body"][0]["For"]["end"] == {"Local": 1}  # for_axis (:1037-1047): counter r + d to extent d
    m = u.lift_reduction("r", "F64", 1, "MaxNum")
    assert skeleton(m["body"]) == [("Let", 3), ("Let", 4), ("For", 1, [("Load", 2, ("buf", 0)), ("Let", 5),
                                                                      *_num_extremum(3, 4)]),
                                   ("Store", ("buf", 1))]


def test_launched_reduction_skeleton_follows_block_reduce():
    """lift_reduction_opdef_launched (block_reduce.rs:50-93): the row's Lets, the thread's strided slice
    of the reduced axis (:278-288), publish (:191-206), a Barrier, log2(block) rounds of `If tid < s`
    (load the partner's partial and flag, fold, publish) each followed by a Barrier (:210-247), thread
    0's store (:292-307), inside the block-strided kept loop (:312-338); locals red and partner_have
    after the serial layout."""
    k = u.lift_reduction("r", "F32", 2, "Max", axes=(1,), launch=(4, 2))
    params, locals_ = _sig(k)
    assert locals_ == ["I32"] * 4 + ["F32", "F64", "I32", "F64", "F32", "I32"]
    rnd = ("If", [("Load", 7, ("shared", 0)), ("Load", 9, ("shared", 1)), ("If", _float_extremum(5, 6), []),
                  ("Store", ("shared", 0)), ("Store", ("shared", 1))], [])
    row = [("Let", 5), ("Let", 6),
           ("For", 3, [("Load", 4, ("buf", 0)), ("Let", 7), *_float_extremum(5, 6)]),
           ("Store", ("shared", 0)), ("Store", ("shared", 1)), ("Barrier",),
           rnd, ("Barrier",), rnd, ("Barrier",),
           ("If", [("Store", ("buf", 1))], [])]
    assert skeleton(k["body"]) == [("For", 2, row)]
    outer = k["body"][0]["For"]
    assert outer["start"] == {"Cast": [{"Exec": {"BlockIdx": 0}}, {"to": "I32", "round": "NearestEven", "sat": "Wrap"}]}
    inner = outer["body"][2]["For"]
    assert inner["start"]["Cast"][0] == {"Exec": {"ThreadIdx": 0}}
    assert inner["step"]["Cast"][0] == {"Exec": {"BlockDim": 0}}
    # no kept axis: the row under `if BlockIdx == 0` (:314-323); Sum publishes no flag
    a = u.lift_reduction("r", "F32", 1, "Sum", launch=(2, 3))
    sk = skeleton(a["body"])
    assert len(sk) == 1 and sk[0][0] == "If"
    assert sk[0][1][:3] == [("Let", 3), ("Let", 4), ("For", 1, [("Load", 2, ("buf", 0)), ("Let", 5), ("Assign", 3)])]
    assert sk[0][1][3:] == [("Store", ("shared", 0)), ("Barrier",),
                            ("If", [("Load", 5, ("shared", 0)), ("Assign", 3), ("Store", ("shared", 0))], []),
                            ("Barrier",), ("If", [("Store", ("buf", 1))], [])]


def test_serial_scan_skeleton_follows_kernel_lift():
    """lift_scan_opdef (kernel_lift.rs:504-519): the kept loops around scan_row (:631-660: Let acc, Let
    have, the scanned loop) around scan_pass (:548-576: loads, val, then the fold and the write, the
    write first for an exclusive scan; a Mean also counts in `have`)."""
    inc = u.lift_scan("s", "I32", 2, "Sum")
    assert skeleton(inc["body"]) == [
        ("For", 2, [("Let", 5), ("Let", 6),
                    ("For", 3, [("Load", 4, ("buf", 0)), ("Let", 7), ("Assign", 5), ("Store", ("buf", 1))])])]
    exc = u.lift_scan("s", "F64", 2, "Mean", axis=0, exclusive=True, reverse=True)
    assert skeleton(exc["body"]) == [
        ("For", 3, [("Let", 5), ("Let", 6),
                    ("For", 2, [("Load", 4, ("buf", 0)), ("Let", 7), ("Store", ("buf", 1)), ("Assign", 5),
                                ("Assign", 6)])])]
    f = exc["body"][0]["For"]["body"][2]["For"]
    i32 = lambda v: {"ConstInt": [v, "I32"]}  # noqa: E731
    assert f["start"] == {"Sub": [{"Local": 0}, i32(1)]} and f["end"] == i32(-1) and f["step"] == i32(-1)


def test_scan_with_a_pre_and_a_post_follows_kernel_lift():
    """lift_scan_opdef with a pre-map and a fused post: scan_loads (kernel_lift.rs:530-545) loads every
    input, then `val = up(pre)` with Input(k) bound to loaded local 2r + k; scan_write (:578-602) lets
    `red` (local 2r + n + 3) hold the prefix rounded once and stores the post with Reduced(0) bound to
    `red` and Input(k) to the loaded locals; `red` is declared after the serial layout (:514-517).  The
    launched lift's phase 1 (fold_only, scan_launched.rs:223-235) and phase 3 take the same loads and
    pre, and only phase 3 writes."""
    from unpopped_amd import expr as X

    x0, x1, r0 = X.input(0), X.input(1), X.reduced(0)
    k = u.lift_scan("s", "F32", 2, "Sum", n_inputs=2, pre=x0 * x1, post=r0 - x0)
    params, locals_ = _sig(k)
    assert params == [("in0", "Buffer", 2), ("in1", "Buffer", 2), ("out", "Buffer", 2), ("n0", "Scalar", 0),
                      ("n1", "Scalar", 1)]
    assert locals_ == ["I32"] * 4 + ["F32", "F32", "F64", "I32", "F64", "F32"]
    assert skeleton(k["body"]) == [
        ("For", 2, [("Let", 6), ("Let", 7),
                    ("For", 3, [("Load", 4, ("buf", 0)), ("Load", 5, ("buf", 1)), ("Let", 8), ("Assign", 6),
                                ("Let", 9), ("Store", ("buf", 2))])])]
    inner = k["body"][0]["For"]["body"][2]["For"]["body"]
    assert inner[2]["Let"]["init"] == {"Cast": [{"Mul": [{"Local": 4}, {"Local": 5}]},
                                               {"to": "F64", "round": "NearestEven", "sat": "Wrap"}]}
    assert inner[4]["Let"]["init"]["Cast"][0] == {"Local": 6}  # red: the F64 prefix cast down once
    assert inner[5]["Store"]["value"] == {"Sub": [{"Local": 9}, {"Local": 4}]}
    # exclusive: the write (Let red, Store) before the fold
    e = u.lift_scan("s", "F64", 1, "Max", exclusive=True, n_inputs=2, pre=x0 - x1, post=r0 * 2.0)
    body = skeleton(e["body"])
    assert body[:2] == [("Let", 4), ("Let", 5)]
    loop = body[2][2]
    assert loop[:4] == [("Load", 2, ("buf", 0)), ("Load", 3, ("buf", 1)), ("Let", 6), ("Let", 7)]
    assert loop[4] == ("Store", ("buf", 2))
    # launched: phase 1 and phase 3 both load both inputs and take the same pre
    la = u.lift_scan("s", "F32", 1, "Sum", n_inputs=2, pre=x0 * x1, post=r0 - x0, launch=(4, 2))
    lets = []

    def walk(x):
        if isinstance(x, dict):
            if "Let" in x and x["Let"]["local"] == 6:  # val = 2r + n + 2
                lets.append(x["Let"]["init"])
            for v in x.values():
                walk(v)
        elif isinstance(x, list):
            for v in x:
                walk(v)

    walk(la["body"])
    assert len(lets) == 2 and lets[0] == lets[1]
    stores = json.dumps(la["body"]).count('"Logical": {"buffer": 2')
    assert stores == 1


def test_gather_skeleton_follows_the_gather_lift():
    """lift_gather_opdef (gather.rs:184-232): locals extents, counters, the loaded data and index, the
    source extent (a Scalar parameter) and the clamped index; each cell loads its index, lets the
    clamp, and guards the data load and store by `raw < 0` then `raw >= extent` (ZeroFill stores zero
    in both out-of-range arms, Skip nothing, Clamp is unguarded)."""
    k = u.lift_gather("g", "Bf16", 2, "I32", oob="ZeroFill")
    params, locals_ = _sig(k)
    assert params == [("in0", "Buffer", 2), ("in1", "Buffer", 2), ("out", "Buffer", 2), ("n0", "Scalar", 0),
                      ("n1", "Scalar", 1), ("src_extent", "Scalar", 6)]
    assert locals_ == ["I32"] * 4 + ["Bf16", "I32", "I32", "I32"]
    compute = [("Load", 4, ("buf", 0)), ("Store", ("buf", 2))]
    zero = [("Store", ("buf", 2))]
    cell = [("Load", 5, ("buf", 1)), ("Let", 6 + 1), ("If", zero, [("If", zero, compute)])]
    assert skeleton(k["body"]) == [("For", 2, [("For", 3, cell)])]
    load = k["body"][0]["For"]["body"][0]["For"]["body"][2]["If"]["els"][0]["If"]["els"][0]["Load"]
    assert load["place"]["Logical"]["coords"] == [{"Local": 7}, {"Local": 3}]  # place_at (:103-113)
    c = u.lift_gather("g", "Bf16", 2, "I32", oob="Clamp", axis=1)
    cl = c["body"][0]["For"]["body"][0]["For"]["body"]
    assert skeleton(cl) == [("Load", 5, ("buf", 1)), ("Let", 7), *compute]
    assert cl[2]["Load"]["place"]["Logical"]["coords"] == [{"Local": 2}, {"Local": 7}]


# ---------------------------------------------------------------------------------------
# The shared launch_cases() corpus (launch_cases.rs:137-180): launched elementwise lifts
# ---------------------------------------------------------------------------------------

from tests.launch_corpus import corpus_args, elementwise_launched, launch_cases, over_inputs  # noqa: E402


@pytest.mark.parametrize("case", launch_cases(), ids=lambda c: c[0])
def test_launch_cases_corpus_lowers_and_runs_on_the_c_leg(case):
    """Each launch_cases() kernel is lowered by lower_kernel as the launched elementwise lift: the lift
    restated here builds the same tree (kernel_lift.rs:96-153), the interface names the lift and the
    kernel's declared launch, and the source compiles for gfx950.  On the corpus's own inputs
    (launch_cases.rs:72-99) the C99 leg agrees with the oracle within the case's ulps
    (launch_cases.rs:14-27)."""
    from oracle import cpuc

    name, dtype, shape, (block, grid), ulps, body, _ = case
    k = elementwise_launched(name, dtype, len(shape), body, block, grid)
    r = len(shape)
    b_in = over_inputs(body, r)
    assert u.lift_elementwise(name, dtype, r, b_in, n_inputs=2, launch=(block, grid)) == k
    g = u.HipBackend().lower_kernel(k)
    assert g.interface["lift"] == "lift_elementwise_opdef_launched"
    assert g.interface["form"] == "elementwise" and g.interface["dtype"] == dtype
    assert g.interface["declared_launch"]["block"] == [block, 1, 1]
    assert [e["symbol"][len(g.name):] for e in g.interface["entries"]] == ["_v", "_s", "_e"]
    u.HipCompiler().compile(g.source, g.name)
    x, y, out = corpus_args(dtype, shape)
    want = oracle.elementwise([x, y], b_in, dtype)
    assert want.any(), "the expected output is not the zeroed buffer (launch_cases.rs:196-203)"
    assert cpuc.run(k, x, y, out, *shape) == cpuc.OK
    if ulps == 0:
        assert out.tobytes() == want.tobytes()
    else:
        ia, ib = out.view(np.int32).astype(np.int64), want.view(np.int32).astype(np.int64)
        assert (np.abs(ia - ib) <= ulps).all()


import numpy as np  # noqa: E402

import oracle  # noqa: E402


# ---------------------------------------------------------------------------------------
# Schedules and Backend::lower_variants (backend.rs:204-309, 786-807)
# ---------------------------------------------------------------------------------------

def test_form_variants_name_the_schedules_and_their_fidelity():
    """Each cell's default is the serial schedule (the sequential fold's bits); the device schedules
    follow with their honest fidelity: bit-identical for integer folds, deterministically divergent for
    a float reduction (a fixed device order) and for a float scan's fixed schedule (the look-back's
    association fixed by the tiling), which comes before the nondeterministic look-back (the carry's
    association depends on timing).  Forms whose schedules agree list one."""
    b = u.HipBackend()

    def summary(**form):
        return [(v["tag"], v["fidelity"], v["schedule"]) for v in b.form_variants(**form)]

    assert summary(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(1,)) == [
        ("serial", "BitIdentical", "serial"), ("device", "DeterministicallyDivergent", "device")]
    assert summary(kind="reduction", dtype="I64", rank=3, op="Xor", axes=(0, 2)) == [
        ("serial", "BitIdentical", "serial"), ("device", "BitIdentical", "device")]
    assert summary(kind="reduction", dtype="F32", rank=2, op="Prod", axes=(1,)) == [("serial", "BitIdentical", "serial")]
    assert summary(kind="scan", dtype="F32", rank=1, op="Sum") == [
        ("serial", "BitIdentical", "serial"), ("fixed", "DeterministicallyDivergent", "fixed"),
        ("device", "Nondeterministic", "device")]
    assert summary(kind="scan", dtype="I32", rank=1, op="Sum") == [
        ("serial", "BitIdentical", "serial"), ("device", "BitIdentical", "device")]
    assert summary(kind="scan", dtype="F64", rank=2, op="Sum", axes=(0,)) == [("serial", "BitIdentical", "serial")]
    for form in (dict(kind="gather", dtype="Bf16", rank=2), dict(kind="dequant4"),
                 dict(kind="row_reduce2", dtype="F32", rank=2), dict(kind="dequant_gemm", dtype="I8", group=128)):
        assert summary(**form) == [("device", "BitIdentical", "device")], form
    vs = b.form_variants(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(1,))
    assert vs[0]["kernel"].interface["schedule"] == "serial"
    assert "serial lift's own order" in vs[0]["kernel"].interface["fidelity_notes"][0]
    # refusals are those of lower_form
    with pytest.raises(_lib.UnpError) as e:
        b.form_variants(kind="reduction", dtype="F32", rank=2, op="Xor")
    assert e.value.kind == "UnsupportedOp" or e.value.kind == "UnsupportedKernel"


def test_fixed_schedule_lowers_a_float_scan_apart_and_other_forms_unchanged():
    """The fixed schedule changes only a float scan's look-back (the unp_scan_fix_ entries, fidelity
    notes saying so, and that the entry, which the row length and alignment pick, fixes the tile size);
    forms whose device schedule is already fixed lower the same source on it."""
    b = u.HipBackend()
    g = b.lower_form("scan", "F32", 1, "Sum", schedule="fixed")
    assert g.name == "unp_scan_fix_incl_sum_f32" and g.interface["schedule"] == "fixed"
    assert "same bits on every launch" in g.interface["fidelity_notes"][0]
    assert "for one entry" in g.interface["fidelity_notes"][0]
    flag = ", true>(in, out, rows, cols"  # the scan templates' FIXED argument
    assert g.source.count(flag) == 2  # the staged and the register entry
    assert flag not in b.lower_form("scan", "F32", 1, "Sum").source
    for form in (dict(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(1,)),
                 dict(kind="scan", dtype="I32", rank=1, op="Sum"),
                 dict(kind="gather", dtype="Bf16", rank=2)):
        assert b.lower_form(schedule="fixed", **form).source == b.lower_form(**form).source, form


def test_lower_kernel_takes_the_fixed_schedule_for_float_scans():
    """A lifted float scan lowers the fixed schedule (the reference's launched scan is reproducible,
    kernel_lift/scan_launched.rs:22-27), with a pre-map too; an integer scan and a float reduction lower
    their device schedule, which is already the same every launch.  The nondeterministic look-back is
    reached only through lower_form(schedule="device")."""
    from unpopped_amd import expr as X

    b = u.HipBackend()
    g = b.lower_kernel(u.lift_scan("s", "F32", 1, "Sum"))
    assert g.interface["schedule"] == "fixed" and g.name.startswith("unp_scan_fix_")
    assert "not reproducible" not in " ".join(g.interface["fidelity_notes"])
    gx = b.lower_kernel(u.lift_scan("s", "F64", 2, "Sum", n_inputs=2, pre=X.input(0) * X.input(1)))
    assert gx.interface["schedule"] == "fixed" and gx.name.startswith("unp_xscan_fix_")
    assert "same bits on every launch" in gx.interface["fidelity_notes"][0]
    assert ", true>(in, out, rows, cols" in gx.source
    assert b.lower_kernel(u.lift_scan("s", "I32", 1, "Sum")).interface["schedule"] == "device"
    dev = b.lower_form("scan", "F32", 1, "Sum", schedule="device")
    assert dev.interface["schedule"] == "device" and "Not reproducible" in dev.interface["fidelity_notes"][0]


def test_schedules_a_form_does_not_have_are_refused():
    b = u.HipBackend()
    with pytest.raises(_lib.UnpError) as e:
        b.lower_form("row_reduce2", "F32", 2, schedule="serial")
    assert e.value.kind == "UnsupportedSchedule"
    f = b.form("reduction", "F32", 2, "Sum")
    f.schedule = 7
    out, err = C.c_void_p(), _lib.Error()
    assert _lib.lib().unp_hip_lower_form(C.byref(f), C.byref(out), C.byref(err)) == 2  # UNSUPPORTED_SCHEDULE
    # the serial schedule of a gather or a dequant is its one kernel
    assert (b.lower_form("gather", "Bf16", 2, schedule="serial").source
            == b.lower_form("gather", "Bf16", 2).source)


def test_general_gather_lift_follows_the_gather_lift():
    """lift_gather_opdef in general (gather.rs:35-101, signature :239-258, cell :184-232): the index
    input's own dtype, src_extent after the extents, locals per input then src_extent and the clamp;
    the cell loads the index, lets the clamp, and under the guards loads every other input (the
    gathered one at the clamped coordinate) before the store of the body."""
    from unpopped_amd import expr as X

    k = u.lift_gather("g", "F32", 2, "I64", oob="ZeroFill", n_inputs=3, data=2, index=0,
                      body=X.input(2) * X.input(1))
    params, locals_ = _sig(k)
    assert params == [("in0", "Buffer", 2), ("in1", "Buffer", 2), ("in2", "Buffer", 2), ("out", "Buffer", 2),
                      ("n0", "Scalar", 0), ("n1", "Scalar", 1), ("src_extent", "Scalar", 7)]
    assert [p["kind"]["Buffer"]["elem"] for p in k["params"][:3]] == ["I64", "F32", "F32"]
    assert locals_ == ["I32"] * 4 + ["I64", "F32", "F32", "I64", "I64"]
    compute = [("Load", 5, ("buf", 1)), ("Load", 6, ("buf", 2)), ("Store", ("buf", 3))]
    zero = [("Store", ("buf", 3))]
    cell = [("Load", 4, ("buf", 0)), ("Let", 8), ("If", zero, [("If", zero, compute)])]
    assert skeleton(k["body"]) == [("For", 2, [("For", 3, cell)])]
    inner = k["body"][0]["For"]["body"][0]["For"]["body"][2]["If"]["els"][0]["If"]["els"]
    assert inner[1]["Load"]["place"]["Logical"]["coords"] == [{"Local": 8}, {"Local": 3}]
    assert inner[2]["Store"]["value"] == {"Mul": [{"Local": 6}, {"Local": 5}]}
    g = u.HipBackend().lower_kernel(k)
    assert g.interface["inputs"] == 3 and g.interface["index_slot"] == 0 and g.interface["data_slot"] == 2
    # a body reading a local that is no input, or a body at an integer dtype, is refused
    bad = json.dumps(k).replace('{"Mul": [{"Local": 6}, {"Local": 5}]}', '{"Mul": [{"Local": 6}, {"Local": 1}]}')
    with pytest.raises(_lib.UnpError) as e:
        u.HipBackend().lower_kernel(bad)
    assert e.value.kind == "UnsupportedKernel"
    ki = u.lift_gather("g", "I32", 2, "I32", n_inputs=3, body=X.input(0) * X.input(2))
    with pytest.raises(_lib.UnpError) as e:
        u.HipBackend().lower_kernel(ki)
    assert e.value.kind == "UnsupportedKernel"
