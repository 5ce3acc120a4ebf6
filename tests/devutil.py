"""Moving reference-layout data to and from device tensors through the C-ABI."""
import ctypes as C

import numpy as np

import oracle_lib as OL
from nc_pkg import nc


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


class DevAct:
    """An activation tensor [rows, cols] on the device, filled from reference bytes."""

    def __init__(self, ref_bytes, dtype, rows, cols):
        L = nc.lib()
        self.dtype, self.rows, self.cols = dtype, rows, cols
        self.pitch = L.nc_act_pitch(dtype, cols)
        host = np.zeros(rows * self.pitch, np.uint8)
        src = np.ascontiguousarray(ref_bytes).view(np.uint8)
        nc.check(L.nc_act_from_reference(ptr(src), ptr(host), dtype, rows, cols), "act_from_reference")
        self.buf = nc.DeviceBuffer(rows * self.pitch)
        self.buf.upload(host)
        self.t = nc.Tensor(self.buf.ptr, None, dtype, rows, cols, self.pitch)

    @classmethod
    def empty(cls, dtype, rows, cols):
        return cls(np.zeros(rows * OL.row_bytes(dtype, cols), np.uint8), dtype, rows, cols)

    def ref(self):
        host = np.zeros(self.rows * self.pitch, np.uint8)
        self.buf.download(host)
        out = np.zeros(self.rows * OL.row_bytes(self.dtype, self.cols), np.uint8)
        nc.check(nc.lib().nc_act_to_reference(ptr(host), ptr(out), self.dtype, self.rows, self.cols), "act_to_ref")
        return out.reshape(self.rows, -1)


class DevWeight:
    """A weight [rows, cols] on the device from its reference payload bytes."""

    def __init__(self, ref_bytes, dtype, rows, cols):
        L = nc.lib()
        cb, db = C.c_size_t(), C.c_size_t()
        nc.check(L.nc_weight_bytes(dtype, rows, cols, C.byref(cb), C.byref(db)), "weight_bytes")
        codes = np.zeros(cb.value, np.uint8)
        deltas = np.zeros(max(db.value, 2), np.uint8)
        src = np.ascontiguousarray(ref_bytes).view(np.uint8)
        nc.check(L.nc_weight_from_reference(ptr(src), dtype, rows, cols, ptr(codes), ptr(deltas)), "weight_from_ref")
        self.cbuf = nc.DeviceBuffer(cb.value)
        self.cbuf.upload(codes)
        self.dbuf = nc.DeviceBuffer(max(db.value, 2))
        self.dbuf.upload(deltas)
        self.t = nc.Tensor(self.cbuf.ptr, self.dbuf.ptr if db.value else None, dtype, rows, cols, 0)


def dev_array(a):
    b = nc.DeviceBuffer(a.nbytes)
    b.upload(np.ascontiguousarray(a))
    return b


def sync():
    nc.check(nc.lib().nc_synchronize(), "synchronize")
