"""Calls into the library's C ABI with its kernels run by the CPU emulator
(tests/emu, script mode of emu_driver): buffers and calls are written to a
file, the driver makes the calls in order with one context, and the
buffers marked for output come back as numpy arrays.  Test infrastructure.

    s = EmuScript(driver)
    leaf = s.dev(leaf_array)                 # hipMalloc'd copy
    out = s.out(n * 4)                       # zeroed device bytes, returned
    s.call("rfxp_set_forest", CTX, leaf, 1, n, ...)
    st = s.run(tmp_path)                     # statuses of the calls
    out.array(np.int32)

Arguments: CTX (the context), Python int / numpy integer (integer slot),
float / numpy floating (real slot), a buffer or buffer.at(byte offset)
(pointer), None (NULL).  The driver casts each slot to the parameter type
include/rfx_prox.h declares."""
import os
import struct
import subprocess

import numpy as np

CTX = object()


class Buf:
    def __init__(self, idx, nbytes, data, host, want):
        self.idx, self.nbytes, self.data, self.host, self.want = idx, nbytes, data, host, want
        self.result = None
        self.off = 0

    def at(self, off):
        v = Buf.__new__(Buf)
        v.__dict__.update(self.__dict__)
        v.off = int(off)
        v.base = self
        return v

    def array(self, dtype, shape=None):
        b = getattr(self, "base", self)
        assert b.result is not None, "buffer not returned (want=False) or script not run"
        a = np.frombuffer(b.result, dtype)
        return a if shape is None else a.reshape(shape)


class EmuScript:
    def __init__(self, driver):
        self.driver = driver
        self.bufs = []
        self.calls = []

    def _buf(self, nbytes, data, host, want):
        b = Buf(len(self.bufs), int(nbytes), data, host, want)
        self.bufs.append(b)
        return b

    def dev(self, arr, want=False):
        a = np.ascontiguousarray(arr)
        return self._buf(a.nbytes, a.tobytes(), False, want)

    def host(self, arr, want=False):
        a = np.ascontiguousarray(arr)
        return self._buf(a.nbytes, a.tobytes(), True, want)

    def out(self, nbytes, host=False):
        return self._buf(nbytes, None, host, True)

    def call(self, name, *args):
        self.calls.append((name, args))

    def run(self, tmp_path, timeout=900, env_extra=None):
        inp, outp = os.path.join(str(tmp_path), "script.bin"), os.path.join(str(tmp_path), "script.out")
        with open(inp, "wb") as f:
            f.write(struct.pack("<ii", 6, len(self.bufs)))
            for b in self.bufs:
                f.write(struct.pack("<iiqi", int(b.host), int(b.want), b.nbytes, int(b.data is not None)))
                if b.data is not None:
                    f.write(b.data)
            f.write(struct.pack("<i", len(self.calls)))
            for name, args in self.calls:
                nb = name.encode()
                f.write(struct.pack("<i", len(nb)) + nb + struct.pack("<i", len(args)))
                for a in args:
                    if a is CTX:
                        f.write(struct.pack("<iqq", 4, 0, 0))
                    elif a is None:
                        f.write(struct.pack("<iqq", 3, 0, 0))
                    elif isinstance(a, Buf):
                        f.write(struct.pack("<iqq", 2, a.idx, a.off))
                    elif isinstance(a, (bool, int, np.integer)):
                        f.write(struct.pack("<iqq", 0, int(a), 0))
                    elif isinstance(a, (float, np.floating)):
                        f.write(struct.pack("<idq", 1, float(a), 0))
                    else:
                        raise TypeError(f"argument {a!r} of {name}")
        env = dict(os.environ, ASAN_OPTIONS="detect_stack_use_after_return=0:detect_leaks=0:abort_on_error=1",
                   **(env_extra or {}))
        r = subprocess.run(["timeout", "-k", "10", str(timeout), self.driver, inp, outp], capture_output=True,
                           text=True, env=env)
        assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-6000:]
        raw = open(outp, "rb").read()
        status, n = struct.unpack_from("<ii", raw, 0)
        assert status == 0, (status, r.stderr[-2000:])
        results = list(struct.unpack_from(f"<{n}q", raw, 8))
        assert len(results) == len(self.calls) and -999999 not in results, (results, r.stderr[-2000:])
        off = 8 + 8 * n
        for b in self.bufs:
            if b.want:
                b.result = raw[off:off + b.nbytes]
                off += b.nbytes
        self.stderr = r.stderr
        return results
