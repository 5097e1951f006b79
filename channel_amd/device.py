"""Host-side handle on the C-ABI: a context, device buffers, checked calls.

Mirrors the reference's GpuContext / GpuBuffer (src/gpu/context.zig,
src/gpu/buffer.zig) with explicit uploads and downloads in place of
host-mapped UMA slices.  Errors surface as ChannelError carrying the
reference-style status name (NoDevice, BatchTooLarge, ...).
"""
import ctypes

import numpy as np

from ._abi import ChannelError, c_f32, c_int, c_void_p, lib


class Buffer:
    """A device allocation owned by a Context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = c_void_p()
        ctx._check("chn_alloc", lib.chn_alloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def offset(self, nbytes):
        """Raw device address nbytes into this buffer."""
        if nbytes < 0 or nbytes > self.nbytes:
            raise ValueError("offset outside buffer")
        return self.ptr + int(nbytes)

    def free(self):
        if self.ptr is not None and self.ctx.handle is not None:
            self.ctx._check("chn_free", lib.chn_free(self.ctx.handle, self.ptr))
        self.ptr = None

    @property
    def _as_parameter_(self):
        return c_void_p(self.ptr)


class Recording:
    """A recorded sequence of calls (chn_record_begin .. chn_record_end), the
    reference's pre-recorded command buffer; submit() enqueues it again."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle

    def submit(self):
        self.ctx._check("chn_submit", lib.chn_submit(self.ctx.handle, self.handle))

    def free(self):
        if self.handle is not None:
            lib.chn_recording_free(self.handle)
            self.handle = None


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, Buffer):
        return a.ptr
    return int(a)


class Context:
    """GpuContext.init equivalent: one HIP device, one stream."""

    def __init__(self, device=0):
        h = c_void_p()
        rc = lib.chn_init(int(device), ctypes.byref(h))
        if rc != 0:
            raise ChannelError("chn_init", rc, lib.chn_last_error(None).decode())
        self.handle = h.value
        self._bufs = []
        self._recs = []

    @property
    def device_name(self):
        """GpuContext.device_name: the device's name and gfx target."""
        return lib.chn_device_name(self.handle).decode()

    # -- plumbing -----------------------------------------------------
    def _check(self, fn, rc):
        if rc != 0:
            msg = lib.chn_last_error(self.handle).decode() if self.handle else ""
            raise ChannelError(fn, rc, msg)
        return rc

    def call(self, fn, *args):
        """Call a chn_* compute entry with Buffers/ints/floats; raise on error."""
        f = getattr(lib, fn)
        conv = []
        for a, t in zip(args, f.argtypes[1:]):
            conv.append(_ptr(a) if t is c_void_p else a)
        return self._check(fn, f(self.handle, *conv))

    def bind(self, fn, *args):
        """A zero-argument callable for a chn_* call repeated with fixed
        arguments (converted once), for launch loops where the per-call
        host cost matters."""
        f = getattr(lib, fn)
        conv = tuple(_ptr(a) if t is c_void_p else a for a, t in zip(args, f.argtypes[1:]))
        h = self.handle

        def call():
            rc = f(h, *conv)
            if rc:
                self._check(fn, rc)
        return call

    def alloc(self, nbytes):
        b = Buffer(self, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr, buf=None):
        a = np.ascontiguousarray(arr)
        if buf is None:
            buf = self.alloc(max(a.nbytes, 1))
        if a.nbytes > buf.nbytes:
            raise ValueError("array larger than buffer")
        self._check("chn_upload", lib.chn_upload(self.handle, buf.ptr,
                                                 a.ctypes.data_as(c_void_p), a.nbytes))
        return buf

    def download(self, buf, dtype, count, byte_offset=0):
        out = np.empty(int(count), dtype=dtype)
        src = _ptr(buf) + int(byte_offset)
        self._check("chn_download", lib.chn_download(self.handle, out.ctypes.data_as(c_void_p),
                                                     src, out.nbytes))
        return out

    def zeros(self, nbytes):
        b = self.alloc(nbytes)
        self.fill_u32(b, 0, (nbytes + 3) // 4)
        return b

    def fill_u32(self, buf, value, count):
        self._check("chn_fill_u32", lib.chn_fill_u32(self.handle, _ptr(buf), value, int(count)))

    def sync(self):
        self._check("chn_sync", lib.chn_sync(self.handle))

    def timer_start(self):
        self._check("chn_timer_start", lib.chn_timer_start(self.handle))

    def timer_stop(self):
        ms = c_f32()
        self._check("chn_timer_stop", lib.chn_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def record_begin(self):
        """Record the following kernel-level calls instead of running them."""
        self._check("chn_record_begin", lib.chn_record_begin(self.handle))

    def record_end(self):
        """End the recording; returns a Recording to submit() any number of times."""
        h = c_void_p()
        self._check("chn_record_end", lib.chn_record_end(self.handle, ctypes.byref(h)))
        r = Recording(self, h.value)
        self._recs.append(r)
        return r

    def close(self):
        if self.handle is None:
            return
        for r in self._recs:
            r.free()
        self._recs = []
        for b in self._bufs:
            if b.ptr is not None:
                lib.chn_free(self.handle, b.ptr)
                b.ptr = None
        self._bufs = []
        lib.chn_destroy(self.handle)
        self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def device_count():
    n = c_int()
    rc = lib.chn_device_count(ctypes.byref(n))
    if rc != 0:
        raise ChannelError("chn_device_count", rc, lib.chn_last_error(None).decode())
    return n.value
