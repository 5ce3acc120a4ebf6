"""The C-ABI library: loads, exports every declared entry point, and its
host-side layout conversions and argument checks work without a GPU."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle_lib as OL

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gten_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(nc_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_entry_point(nc):
    L = nc.lib()
    names = declared_functions()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_act_layout_roundtrip(nc, oracle):
    L = nc.lib()
    rng = np.random.default_rng(0)
    for dt, cols in [(nc.Q8, 2048), (nc.Q8, 96), (nc.F16, 320), (nc.F32, 64)]:
        rows = 3
        x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
        if dt == nc.Q8:
            ref = np.zeros((rows, OL.row_bytes(dt, cols)), np.uint8)
            for r in range(rows):
                oracle.q8_quantize_row(OL.ptr(x[r]), OL.ptr(ref[r]), cols)
        elif dt == nc.F16:
            ref = x.astype(np.float16).view(np.uint8)
        else:
            ref = x.view(np.uint8)
        pitch = L.nc_act_pitch(dt, cols)
        assert pitch % 16 == 0
        dev = np.zeros(rows * pitch, np.uint8)
        nc.check(L.nc_act_from_reference(OL.ptr(ref), OL.ptr(dev), dt, rows, cols))
        back = np.zeros_like(ref)
        nc.check(L.nc_act_to_reference(OL.ptr(dev), OL.ptr(back), dt, rows, cols))
        assert np.array_equal(back, ref)
        if dt == nc.Q8:  # codes first, then the fp16 deltas, per row
            nb = cols // 32
            row0 = dev[:pitch]
            assert np.array_equal(row0[:32], ref[0, 2:34])
            assert np.array_equal(row0[nb * 32:nb * 32 + 2], ref[0, :2])


@pytest.mark.parametrize("dt", [4, 3])  # Q4, Q8
def test_weight_lane_permutation(nc, oracle, dt):
    """Dword k of a repacked block holds exactly the codes of the reference's
    lane k: elements {2k, 2k+1, 2k+8, 2k+9} and the same + 16."""
    L = nc.lib()
    rng = np.random.default_rng(dt)
    rows, cols = 4, 64
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    ref = np.zeros((rows, OL.row_bytes(dt, cols)), np.uint8)
    (oracle.q8_quantize_weights if dt == nc.Q8 else oracle.q4_quantize_weights)(OL.ptr(w), rows * cols // 32,
                                                                               OL.ptr(ref))
    cb, db = C.c_size_t(), C.c_size_t()
    nc.check(L.nc_weight_bytes(dt, rows, cols, C.byref(cb), C.byref(db)))
    codes = np.zeros(cb.value, np.uint8)
    deltas = np.zeros(db.value, np.uint8)
    nc.check(L.nc_weight_from_reference(OL.ptr(ref), dt, rows, cols, OL.ptr(codes), OL.ptr(deltas)))
    bsz = 34 if dt == nc.Q8 else 18
    blocks = ref.reshape(-1, bsz)
    assert np.array_equal(deltas.view(np.uint16), blocks[:, :2].copy().view(np.uint16).reshape(-1))
    per = 32 if dt == nc.Q8 else 16
    for b in range(blocks.shape[0]):
        raw = blocks[b, 2:]
        if dt == nc.Q8:
            elem = raw.view(np.int8).astype(int)
        else:
            elem = np.concatenate([raw >> 4, raw & 15]).astype(int)
        cb_ = codes[b * per:(b + 1) * per]
        for k in range(4):
            lane = [2 * k, 2 * k + 1, 2 * k + 8, 2 * k + 9]
            if dt == nc.Q8:
                assert cb_[8 * k:8 * k + 4].view(np.int8).tolist() == elem[lane].tolist()
                assert cb_[8 * k + 4:8 * k + 8].view(np.int8).tolist() == elem[[e + 16 for e in lane]].tolist()
            else:
                dword = cb_[4 * k:4 * k + 4]
                assert (dword >> 4).tolist() == elem[lane].tolist()
                assert (dword & 15).tolist() == elem[[e + 16 for e in lane]].tolist()


def test_rope_table_is_the_reference_expression(nc, oracle):
    """nc_rope_table's (cos, sin) are what the reference's rotary_emb applies:
    rotating the unit vectors e_j (fp32 rows) gives exactly cos and sin."""
    L = nc.lib()
    n, d_head = 40, 64
    for pct in (1.0, 0.25):
        d_half = int(d_head * pct) // 2
        tab = np.zeros((n, d_half, 2), np.float32)
        nc.check(L.nc_rope_table(n, d_head, pct, OL.ptr(tab)))
        for j in range(d_half):
            x = np.zeros((n, d_head), np.float32)
            x[:, j] = 1.0
            out = np.zeros_like(x)
            oracle.rotary_emb(OL.ptr(x), OL.ptr(out), OL.F32, d_head, d_head, pct, 0, n)
            assert np.array_equal(out[:, j], tab[:, j, 0])
            assert np.array_equal(out[:, j + d_half], tab[:, j, 1])


def test_argument_errors_are_reported(nc):
    L = nc.lib()
    cb, db = C.c_size_t(), C.c_size_t()
    assert L.nc_weight_bytes(nc.Q4, 4, 33, C.byref(cb), C.byref(db)) == -1
    assert b"multiple of 32" in L.nc_last_error()
    x = nc.Tensor(1, None, nc.Q8, 2, 64, 96)
    w = nc.Tensor(1, 1, nc.Q4, 8, 32, 0)
    out = nc.Tensor(1, None, nc.F32, 2, 8, 32)
    assert L.nc_matmul_2d(C.byref(x), C.byref(w), C.byref(out), 0, 2, None) == -1
    assert b"columns" in L.nc_last_error()
    q = nc.Tensor(1, None, nc.Q8, 4, 128, 160)
    k = nc.Tensor(1, None, nc.F16, 4, 64, 128)
    assert L.nc_qkv_attn(C.byref(q), C.byref(k), C.byref(k), C.byref(q), 2, 1, 64, 0, 4, None) == -1
    assert b"dtypes" in L.nc_last_error()
    assert L.nc_debug_spec(-1.0, None) == -1
    assert b"skew" in L.nc_last_error()
    assert L.nc_debug_spec(1.0, None) == 0


def test_kernel_expf_equals_host_libm_exhaustive(nc, oracle):
    """The kernels' expf (evaluated on the host from the same source) equals
    the host glibc expf -- std::exp(float) of the reference -- on all 2^32
    inputs."""
    fn_addr = C.cast(nc.lib().nc_expf_host, C.c_void_p).value
    chk = oracle.lib.or_check_expf_fn
    chk.restype = C.c_int64
    chk.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.POINTER(C.c_int64)]
    first = C.c_int64()
    bad = chk(fn_addr, 0, 1 << 32, C.byref(first))
    assert bad == 0, f"{bad} inputs differ, first bits {first.value:#x}"
