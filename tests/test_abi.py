"""The C-ABI boundary without a GPU: library loads, exports every declared symbol,
struct layouts agree with the header, and the host-built encode tables reproduce
the reference's rounding rules."""

import ctypes
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest
import torch

from adamw4bit_amd import _lib
from adamw4bit_amd import quantization as q
from oracle import reference_step as ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "adamw4bit_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aw4_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), "ctypes signatures and header disagree"
    for name in names:
        assert hasattr(lib, name), name
    assert lib.aw4_abi_version() == _lib.ABI_VERSION


def test_error_path_reports_message():
    # Invalid arguments are rejected on the host before any device work.
    lib = _lib.library()
    rc = lib.aw4_uniforms(1, 2, 16, None, None)  # null output
    assert rc == _lib.EINVAL
    assert b"aw4_uniforms" in lib.aw4_last_error()
    table = np.zeros(1, dtype=_lib.TENSOR)  # null pointers
    with pytest.raises(_lib.HipLibraryError, match="null param"):
        _lib.fused_step(table, 0)
    with pytest.raises(_lib.HipLibraryError, match="null grad"):
        _lib.clip_coefficient(table, 1.0, 64, 64, 0)


def _row(**m2):
    """A well-formed fp32 row with fake (aligned, never dereferenced) addresses: ZIP-SR-like m1
    and the given m2 fields."""
    t = np.zeros(1, dtype=_lib.TENSOR)
    t["param"], t["grad"], t["numel"] = 1 << 20, 2 << 20, 4096
    t["param_dtype"] = t["grad_dtype"] = _lib.F32
    m1 = t["m1"]
    m1["codes"], m1["scales"], m1["codebook"], m1["rounding"] = 3 << 20, 4 << 20, _lib.CB_NF4, _lib.ROUND_RTN
    base = dict(codes=5 << 20, scales=6 << 20, codebook=_lib.CB_DYN4, rounding=_lib.ROUND_LOOKAHEAD_SR,
                la_beta2=0.95, la_fresh_weight=0.05, la_bias=0.05, la_eps=1e-8)
    base.update(m2)
    for k, v in base.items():
        t["m2"][k] = v
    return t


@pytest.mark.parametrize("m2,message", [
    (dict(codebook=_lib.CB_LIN4), "dyn4 m2 only"),
    (dict(flags=_lib.MOMENT_FRESH_PROXY | _lib.MOMENT_PENDING), "FRESH_PROXY and PENDING"),
    (dict(flags=_lib.MOMENT_SAMPLED_READ), "read-back or EDEN"),
    (dict(flags=_lib.MOMENT_EDEN), "read-back or EDEN"),
    (dict(la_bias=0.0), "bias > 0"),
    (dict(la_beta2=1.0), "beta2 in"),
    (dict(flags=_lib.MOMENT_PENDING, values=0), "pending lookahead m2 without"),
    (dict(flags=_lib.MOMENT_PENDING, values=(7 << 20) + 4), "pending lookahead m2 without"),
    (dict(rounding=_lib.ROUND_UPDATE_SR, flags=_lib.MOMENT_PENDING, sr_bias=1.0), "lookahead flags without"),
    (dict(rounding=5), "has rounding 5"),
    (dict(rng_offset=100), "multiple of 128"),
])
def test_lookahead_rows_are_validated_on_the_host(m2, message):
    # check_moment rejects malformed lookahead rows before any device work
    with pytest.raises(_lib.HipLibraryError, match=message):
        _lib.fused_step(_row(**m2), 0)


def test_grad_scale_and_clip_arguments_are_validated_on_the_host():
    t = _row()
    t["flags"] = _lib.TENSOR_GRAD_SCALE  # without an address
    with pytest.raises(_lib.HipLibraryError, match="GRAD_SCALE"):
        _lib.fused_step(t, 0)
    t["grad_scale"] = (8 << 20) + 2  # misaligned
    with pytest.raises(_lib.HipLibraryError, match="GRAD_SCALE"):
        _lib.fused_step(t, 0)
    c = _row()
    c["grad_dtype"] = 7
    with pytest.raises(_lib.HipLibraryError, match="grad dtype"):
        _lib.clip_coefficient(c, 1.0, 64, 128, 0)
    c["grad_dtype"], c["flags"], c["grad"] = _lib.F32, _lib.TENSOR_VEC_ALIGNED, (2 << 20) + 4
    with pytest.raises(_lib.HipLibraryError, match="VEC_ALIGNED"):
        _lib.clip_coefficient(c, 1.0, 64, 128, 0)
    with pytest.raises(_lib.HipLibraryError, match="4-byte aligned"):
        _lib.clip_coefficient(_row(), 1.0, 66, 128, 0)
    lib = _lib.library()
    assert lib.aw4_clip_coefficient(None, 1, 1.0, 64, 128, None) == _lib.EINVAL
    assert lib.aw4_clip_coefficient(_row().ctypes.data, 0, 1.0, 64, 128, None) == _lib.EINVAL
    q = _row()["m2"].copy()
    assert lib.aw4_quantize(1 << 20, 4096, q.ctypes.data, None) == _lib.EINVAL
    assert b"lookahead" in lib.aw4_last_error()


def test_struct_layout_matches_header():
    src = r"""
#include <stddef.h>
#include <stdio.h>
#include "adamw4bit_hip.h"
#define P(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("aw4_moment %zu\naw4_tensor %zu\n", sizeof(aw4_moment), sizeof(aw4_tensor));
  P(aw4_moment, codes) P(aw4_moment, scales) P(aw4_moment, values) P(aw4_moment, draws)
  P(aw4_moment, rng_seed) P(aw4_moment, rng_offset) P(aw4_moment, codebook) P(aw4_moment, rounding)
  P(aw4_moment, flags) P(aw4_moment, sr_bias) P(aw4_moment, sr_bias_rcp) P(aw4_moment, sr_eps)
  P(aw4_moment, la_beta2) P(aw4_moment, la_fresh_weight) P(aw4_moment, la_bias) P(aw4_moment, la_eps)
  P(aw4_tensor, param) P(aw4_tensor, grad) P(aw4_tensor, grad_scale) P(aw4_tensor, numel) P(aw4_tensor, param_dtype)
  P(aw4_tensor, grad_dtype) P(aw4_tensor, flags) P(aw4_tensor, w1) P(aw4_tensor, w2) P(aw4_tensor, decay)
  P(aw4_tensor, step_coef) P(aw4_tensor, bc2_sqrt) P(aw4_tensor, bc2_sqrt_rcp) P(aw4_tensor, eps)
  P(aw4_tensor, m1) P(aw4_tensor, m2) P(aw4_tensor, decay_f64) P(aw4_tensor, step_coef_f64)
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line)
    assert int(got["aw4_moment"]) == _lib.MOMENT.itemsize
    assert int(got["aw4_tensor"]) == _lib.TENSOR.itemsize
    for name, dtype in (("aw4_moment", _lib.MOMENT), ("aw4_tensor", _lib.TENSOR)):
        for field, (_, offset) in dtype.fields.items():
            assert int(got[f"{name}.{field}"]) == offset, (name, field)


def test_header_constants_match_python():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (AW4_[A-Z0-9_]+) (-?(?:0x)?[0-9A-Fa-f]+)\b", text))
    val = {k: int(v, 0) for k, v in consts.items()}
    assert val["AW4_CB_NF4"] == q.CB_NF4 == _lib.CB_NF4
    assert val["AW4_CB_SDYN4"] == q.CB_SDYN4 and val["AW4_CB_DYN4"] == q.CB_DYN4
    assert val["AW4_CB_LIN4"] == q.CB_LIN4 and val["AW4_CB_LIN4_NZ"] == q.CB_LIN4_NZ
    assert val["AW4_ROUND_RTN"] == q.ROUND_RTN == _lib.ROUND_RTN
    assert val["AW4_ROUND_STATE_SR"] == q.ROUND_STATE_SR and val["AW4_ROUND_UPDATE_SR"] == q.ROUND_UPDATE_SR
    assert val["AW4_NUM_LUTS"] == _lib.NUM_LUTS and val["AW4_LUT_HALF"] == _lib.LUT_HALF
    assert val["AW4_LUT_EXP0"] == _lib.LUT_EXP0 and val["AW4_BLOCK"] == _lib.BLOCK
    for name in ("MOMENT_ZERO_FLOOR", "MOMENT_EDEN", "MOMENT_GUARDS", "MOMENT_EXT_DRAWS", "MOMENT_SAMPLED_READ",
                 "MOMENT_READ_RAW_SCALE", "MOMENT_FRESH_PROXY", "MOMENT_PENDING", "ROUND_LOOKAHEAD_SR",
                 "TENSOR_LERP1_LARGE", "TENSOR_LERP2_LARGE", "TENSOR_VEC_ALIGNED", "TENSOR_GRAD_SCALE", "F32", "BF16",
                 "F16"):
        assert val[f"AW4_{name}"] == getattr(_lib, name), name


# ---------------------------------------------------------------------------
# Encode tables: bucket lookup == reference rounding rule
# ---------------------------------------------------------------------------

LUT_CODEBOOKS = [("nf4", q.CB_NF4), ("sdyn4", q.CB_SDYN4), ("dyn4", q.CB_DYN4), ("lin4", q.CB_LIN4),
                 ("lin4_nz", q.CB_LIN4_NZ)]


def lut_eval(tables, lut_id, x):
    """The kernel's lut_index() restated in numpy."""
    u = x.view(np.uint32).astype(np.int64)
    k = ((u & 0x7FFFFFFF) >> 20) - (_lib.LUT_EXP0 - 1)
    k = np.clip(k, 0, _lib.LUT_HALF - 1)
    idx = k + (u >> 31) * _lib.LUT_HALF
    thr = tables[lut_id, idx, 0].view(np.float32)
    return tables[lut_id, idx, 1].astype(np.int64) + (x >= thr)


def lut_level(tables, lut_id, x):
    """Level the kernel reads from the entry: the code's level (round-to-nearest tables) or
    the upper neighbour cb[min(count, 15)] (level-count tables)."""
    u = x.view(np.uint32).astype(np.int64)
    k = np.clip(((u & 0x7FFFFFFF) >> 20) - (_lib.LUT_EXP0 - 1), 0, _lib.LUT_HALF - 1)
    idx = k + (u >> 31) * _lib.LUT_HALF
    e = tables[lut_id, idx]
    up = x >= e[:, 0].view(np.float32)
    return np.where(up, e[:, 3].view(np.float32), e[:, 2].view(np.float32))


def reference_rules(cb: np.ndarray, x: np.ndarray):
    """searchsorted-left count and the round-to-nearest code, via the oracle's torch ops."""
    xt = torch.from_numpy(x)
    cbt = torch.from_numpy(cb)
    idx = torch.searchsorted(cbt, xt, out_int32=True)
    lower, upper, a, b = ref._endpoints(xt, cbt)
    rtn = torch.where((xt - a).abs() < (b - xt).abs(), lower, upper)
    return idx.numpy().astype(np.int64), rtn.numpy().astype(np.int64)


def probe_values(cb: np.ndarray, tables: np.ndarray) -> np.ndarray:
    rng = np.random.default_rng(0)
    pts = [rng.uniform(-1, 1, 200000).astype(np.float32), (rng.uniform(0, 1, 100000) ** 6).astype(np.float32),
           np.array([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30, 2.0 ** -10, -(2.0 ** -10), 1e-45], dtype=np.float32)]
    # every threshold of every table and every level, +-40 ulps
    marks = [cb, tables[:, :, 0].view(np.float32).reshape(-1)]
    for m in marks:
        m = m[np.isfinite(m)].astype(np.float32)
        bits = m.view(np.int32)
        for d in range(-40, 41):
            b = bits + d
            pts.append(b.view(np.float32))
            pts.append((-(m)).astype(np.float32).view(np.int32) + d)
    # bucket edges +-3 ulps
    edges = (np.arange(_lib.LUT_EXP0, _lib.LUT_EXP0 + _lib.LUT_HALF, dtype=np.int64) << 20)
    for d in range(-3, 4):
        e = (edges + d).astype(np.uint32).view(np.float32)
        pts += [e, -e]
    x = np.concatenate([np.asarray(p).view(np.float32) if np.asarray(p).dtype != np.float32 else p for p in pts])
    x = x[np.isfinite(x) & (np.abs(x) <= 1.0)]
    return np.ascontiguousarray(x, dtype=np.float32)


@pytest.mark.parametrize("mode,cb_id", LUT_CODEBOOKS)
def test_encode_tables_reproduce_rounding_rules(mode, cb_id):
    tables = _lib.encode_tables()
    cb = np.array(q.CODEBOOK_VALUES[cb_id], dtype=np.float32)
    x = probe_values(cb, tables)
    count, rtn = reference_rules(cb, x)
    assert np.array_equal(lut_eval(tables, cb_id, x), rtn)                 # round-to-nearest table
    assert np.array_equal(lut_eval(tables, 6 + cb_id, x), count)           # level-count table
    assert np.array_equal(lut_level(tables, 6 + cb_id, x), cb[np.minimum(count, 15)])  # its upper level b
    assert np.array_equal(lut_level(tables, cb_id, x), cb[rtn])            # the level EDEN uses
    if mode == "dyn4":
        floored = np.maximum(rtn, 1)
        assert np.array_equal(lut_eval(tables, 5, x), floored)             # dyn4_nz floor table
        assert np.array_equal(lut_level(tables, 5, x), cb[floored])


@pytest.mark.parametrize("mode,cb_id", LUT_CODEBOOKS)
def test_encode_tables_on_infinite_and_nan_values(mode, cb_id):
    """+-inf and NaN take searchsorted's count and round-to-nearest code too: no table entry
    increments past its bucket's count (a bucket without a change has a NaN threshold).  A NaN x
    reaches the table as the positive quiet NaN (the encode makes it so)."""
    tables = _lib.encode_tables()
    cb = np.array(q.CODEBOOK_VALUES[cb_id], dtype=np.float32)
    x = np.array([np.inf, -np.inf, np.nan, 3e38, -3e38], dtype=np.float32)
    count, rtn = reference_rules(cb, x)
    assert np.array_equal(lut_eval(tables, 6 + cb_id, x), count)
    assert np.array_equal(lut_eval(tables, cb_id, x), rtn)


def test_aten_row_sum_order():
    """The per-block sum order the kernel reproduces (8 lanes x 4 accumulators) is ATen's."""
    gen = torch.Generator().manual_seed(0)
    rows = torch.rand(4000, 128, generator=gen) ** 3
    got = rows.sum(dim=1)
    r = rows.numpy().reshape(-1, 16, 8)
    acc = [r[:, k] + np.float32(0) for k in range(4)]
    for k in range(4):
        for v in (k + 4, k + 8, k + 12):
            acc[k] = (acc[k] + r[:, v]).astype(np.float32)
    a = (((acc[0] + acc[1]).astype(np.float32) + acc[2]).astype(np.float32) + acc[3]).astype(np.float32)
    s = np.zeros(len(rows), dtype=np.float32)
    for lane in range(8):
        s = (s + a[:, lane]).astype(np.float32)
    assert np.array_equal(s, got.numpy())
    # a plausible slip (sequential order) would not match
    seq = np.zeros(len(rows), dtype=np.float32)
    for j in range(128):
        seq = (seq + rows.numpy()[:, j]).astype(np.float32)
    assert not np.array_equal(seq, got.numpy())


def test_aten_elementwise_semantics():
    """ATen CPU facts the kernel's arithmetic relies on: lerp is one fused multiply-add,
    division by a Python scalar is a true fp32 division, addcdiv is p + (v*t1)/t2."""
    gen = torch.Generator().manual_seed(1)
    m = torch.randn(100003, generator=gen) * 1e-3
    g = torch.randn(100003, generator=gen) * 1e-3
    for w in (0.1, 0.05, 0.7):
        got = m.clone().lerp_(g, w).numpy()
        wf = np.float32(w)
        mn, gn = m.numpy(), g.numpy()
        d = (gn - mn).astype(np.float32)
        if abs(wf) < 0.5:
            expect = np.float32(mn.astype(np.float64) + np.float64(wf) * d.astype(np.float64))
        else:
            expect = np.float32(gn.astype(np.float64) + np.float64(wf - np.float32(1)) * d.astype(np.float64))
        assert np.array_equal(got, expect.astype(np.float32)), w
    s = 0.31622776601683794
    a = m.abs()
    assert np.array_equal(a.clone().div_(s).numpy(), a.numpy() / np.float32(s))
    # ATen's CPU sqrt (MKL vector math) is not correctly rounded: results are the correctly
    # rounded square root or 1 ulp below it.  The kernel's parameter update uses the hardware's
    # faithful square root (v_sqrt_f32, within 1 ulp), the same precision class, so values
    # downstream of that square root agree within about 1 ulp per use.
    cr = np.sqrt(a.numpy().astype(np.float64)).astype(np.float32)
    ulps = a.sqrt().numpy().view(np.int32).astype(np.int64) - cr.view(np.int32)
    assert set(np.unique(ulps).tolist()) <= {-1, 0}
    assert np.mean(ulps != 0) < 0.02
    t1, t2 = m.numpy(), np.abs(g.numpy()) + np.float32(1e-3)
    got = torch.from_numpy(np.ones_like(t1)).addcdiv_(m, torch.from_numpy(t2), value=-1e-3).numpy()
    assert np.array_equal(got, np.float32(1) + (np.float32(-1e-3) * t1) / t2)


def test_torch_custom_op_schema_and_argument_checks():
    """The launch is the torch operator adamw4bit_hip::fused_step_: it declares the tensors it
    writes (parameters, moment states) and reads (gradients, draws), and checks its table and
    address references."""
    import torch

    import adamw4bit_amd  # noqa: F401  (registers the operator)

    op = torch.ops.adamw4bit_hip.fused_step_
    schema = str(op.default._schema)
    assert schema.startswith("adamw4bit_hip::fused_step_(Tensor(a0!)[] params, Tensor(a1!)[] states, "
                             "Tensor[] inputs, Tensor table, Tensor refs)")
    refs0 = torch.zeros((0, 11), dtype=torch.int64)
    op([], [], [], torch.zeros(0, dtype=torch.uint8), refs0)  # nothing to launch
    row = _lib.TENSOR.itemsize
    with pytest.raises(ValueError, match="CPU uint8 tensor"):
        op([torch.zeros(4)], [], [], torch.zeros(row, dtype=torch.float32), refs0)
    with pytest.raises(ValueError, match="CPU int64"):
        op([torch.zeros(4)], [], [], torch.zeros(row, dtype=torch.uint8), refs0.to(torch.int32))
    with pytest.raises(ValueError, match="HIP devices only"):
        op([torch.zeros(4)], [], [], torch.zeros(row, dtype=torch.uint8), torch.zeros((1, 11), dtype=torch.int64))
    clip = torch.ops.adamw4bit_hip.clip_coefficient_
    assert str(clip.default._schema).startswith(
        "adamw4bit_hip::clip_coefficient_(Tensor[] grads, Tensor(a1!) out, Tensor table, float max_norm)")
    with pytest.raises(ValueError, match="HIP device"):
        clip([torch.zeros(4)], torch.zeros(2), torch.zeros(row, dtype=torch.uint8), 1.0)


def test_operator_takes_addresses_from_its_tensors():
    """The operator writes each row's address fields from the tensors it receives (reference -1:
    no buffer), so a copy that functionalization hands it is the memory the kernel writes."""
    import torch

    from adamw4bit_amd import _ops

    tensors = [torch.zeros(8), torch.zeros(16, dtype=torch.uint8), torch.zeros(4), torch.ones(8)]
    rows = np.zeros(2, dtype=_lib.TENSOR)
    rows["numel"] = [8, 8]
    refs = np.full((2, len(_ops.ADDRESS_FIELDS)), -1, dtype=np.int64)
    col = {".".join(p): k for k, p in enumerate(_ops.ADDRESS_FIELDS)}
    refs[0, col["param"]], refs[0, col["grad"]], refs[0, col["m1.codes"]], refs[0, col["m1.scales"]] = 0, 3, 1, 2
    refs[1, col["param"]], refs[1, col["m2.values"]] = 3, 0
    rows["param"] = 123  # stale addresses are overwritten
    _ops.resolve_addresses(rows, refs, tensors)
    assert rows["param"][0] == tensors[0].data_ptr() and rows["grad"][0] == tensors[3].data_ptr()
    assert rows["m1"]["codes"][0] == tensors[1].data_ptr() and rows["m1"]["scales"][0] == tensors[2].data_ptr()
    assert rows["param"][1] == tensors[3].data_ptr() and rows["m2"]["values"][1] == tensors[0].data_ptr()
    for path in ("grad_scale", "m1.values", "m1.draws", "m2.codes", "m2.scales", "m2.draws"):
        obj = rows
        for name in path.split("."):
            obj = obj[name]
        assert obj[0] == 0, path
    assert rows["grad"][1] == 0 and rows["m1"]["codes"][1] == 0 and rows["numel"][1] == 8
    with pytest.raises(ValueError, match="outside"):
        _ops.resolve_addresses(rows, np.full_like(refs, 4), tensors)
    with pytest.raises(ValueError, match="contiguous"):
        _ops.resolve_addresses(rows, refs, [torch.zeros(4, 4).t()] + tensors[1:])


def test_plan_step_view_covers_exactly_the_per_step_fields():
    """The launch plan rewrites each step through one fixed view of the table rows; writing
    through it changes the per-step fields and leaves every other byte of the row alone."""
    import numpy as np
    from adamw4bit_amd import _lib
    from adamw4bit_amd.adamw import _STEP_FIELDS, _STEP_WORDS
    T = _lib.TENSOR
    assert _STEP_FIELDS.itemsize == T.itemsize == 296 and _STEP_WORDS.itemsize == 32
    row = np.zeros(2, dtype=T)
    raw = row.view(np.uint8).reshape(2, -1)
    raw[:] = 0xA5
    before = raw.copy()
    view = row.view(_STEP_FIELDS)
    view["grad"] = [11, 12]
    view["grad_scale"] = [13, 14]
    words = np.array([(3, 0.5, 0.25, 0.75, -1e-3, 0.125, 8.0, 1e-8)] * 2, dtype=_STEP_WORDS)
    view["words"] = words.view(np.uint32).reshape(-1, 8)
    view["m2_sr"] = np.array([[1.5, 2.5, 3.5]] * 2, dtype=np.float32).view(np.uint32)
    view["m1_rng_seed"] = [31, 32]
    view["m2_rng_seed"] = [33, 34]
    view["m1_rng_offset"] = [21, 22]
    view["m2_rng_offset"] = [23, 24]
    view["f64"] = [(0.999, -2.5e-4), (0.998, -3.5e-4)]
    assert list(row["grad"]) == [11, 12] and list(row["grad_scale"]) == [13, 14]
    assert list(row["decay_f64"]) == [0.999, 0.998] and list(row["step_coef_f64"]) == [-2.5e-4, -3.5e-4]
    assert list(row["flags"]) == [3, 3]
    for name, value in zip(("w1", "w2", "decay", "step_coef", "bc2_sqrt", "bc2_sqrt_rcp", "eps"),
                           (0.5, 0.25, 0.75, -1e-3, 0.125, 8.0, 1e-8)):
        assert np.all(row[name] == np.float32(value)), name
    assert np.all(row["m2"]["sr_bias"] == 1.5) and np.all(row["m2"]["sr_bias_rcp"] == 2.5)
    assert np.all(row["m2"]["sr_eps"] == 3.5)
    assert list(row["m1"]["rng_offset"]) == [21, 22] and list(row["m2"]["rng_offset"]) == [23, 24]
    assert list(row["m1"]["rng_seed"]) == [31, 32] and list(row["m2"]["rng_seed"]) == [33, 34]
    # every byte outside those fields is untouched
    written = np.zeros(T.itemsize, dtype=bool)
    for name in _STEP_FIELDS.names:
        dt, off = _STEP_FIELDS.fields[name][:2]
        written[off:off + dt.itemsize] = True
    assert written.sum() == 8 + 8 + 32 + 12 + 4 * 8 + 16
    assert np.array_equal(raw[:, ~written], before[:, ~written])


def test_noalloc_step_rejects_tables_beyond_its_area():
    """aw4_fused_step_noalloc checks its rows and the size of their launch tables before any
    device work: tables beyond AW4_NOALLOC_TABLE_BYTES fail with a clear error (no GPU needed)."""
    lib = _lib.library()
    n = _lib.NOALLOC_TABLE_BYTES // (_lib.TENSOR.itemsize + 8) + 8
    rows = np.zeros(n, dtype=_lib.TENSOR)
    rows["param"], rows["grad"], rows["numel"] = 1 << 20, 2 << 20, 100  # fp32-state rows: never touched
    rows["m1"]["values"], rows["m2"]["values"] = 3 << 20, 4 << 20
    rows["m1"]["rounding"] = rows["m2"]["rounding"] = _lib.ROUND_FP32
    rc = lib.aw4_fused_step_noalloc(rows.ctypes.data, len(rows), None)
    assert rc == _lib.EINVAL
    assert b"more than its 1048576-byte table area" in lib.aw4_last_error()
    rows["numel"][7] = 0
    assert lib.aw4_fused_step_noalloc(rows.ctypes.data, len(rows), None) == _lib.EINVAL
    assert b"tensor 7: numel 0" in lib.aw4_last_error()


def test_step_rejects_unknown_dtypes_and_scaled_float64_gradients():
    """Rows are checked before any device work (no GPU needed): a dtype code outside
    AW4_F32/BF16/F16/F64 fails, and so does a float64 gradient with GRAD_SCALE or GRAD_UNSCALE (the
    prologue's coefficients are fp32 products of fp32/bf16/fp16 gradients)."""
    lib = _lib.library()
    rows = np.zeros(1, dtype=_lib.TENSOR)
    rows["param"], rows["grad"], rows["numel"], rows["grad_scale"] = 1 << 20, 2 << 20, 256, 5 << 20
    rows["param_dtype"] = rows["grad_dtype"] = _lib.F64
    rows["m1"]["values"], rows["m2"]["values"] = 3 << 20, 4 << 20
    rows["m1"]["rounding"] = rows["m2"]["rounding"] = _lib.ROUND_FP32
    for flag in (_lib.TENSOR_GRAD_SCALE, _lib.TENSOR_GRAD_UNSCALE):
        rows["flags"] = flag
        assert lib.aw4_fused_step(rows.ctypes.data, 1, None) == _lib.EINVAL
        assert b"tensor 0: GRAD_SCALE/GRAD_UNSCALE with a float64 gradient" in lib.aw4_last_error()
    rows["flags"] = 0
    rows["param_dtype"] = 4
    assert lib.aw4_fused_step(rows.ctypes.data, 1, None) == _lib.EINVAL
    assert b"tensor 0: dtype 4" in lib.aw4_last_error()
