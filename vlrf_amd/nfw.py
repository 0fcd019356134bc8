"""NFW weight files: the reference's format (include/model/weights.hpp:58-62,
289-339; tools/converter/nfw_writer.py:11-44) with this backend's version 3,
which adds GGUF block payloads (dtype 2 = Q4_0, 8 = Q8_0, GGML's numbers).

Reading goes through the library's C++ parser (vlrf_nfw_*, host only: no
device is touched); writing is a plain byte layout, as the reference's
converter writes it.
"""
import ctypes as C
import struct

import numpy as np

from ._lib import check, lib

MAGIC = 0x4E465746
F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}


class Blocks:
    """A block-quantized tensor: logical shape (rows, ..., cols), GGUF blocks
    of 32 consecutive elements in row-major order."""

    def __init__(self, dtype, shape, data):
        if dtype not in BLOCK_BYTES:
            raise ValueError(f"block dtype {dtype} is not Q8_0 or Q4_0")
        numel = int(np.prod(shape))
        if shape[-1] % 32 or len(data) != numel // 32 * BLOCK_BYTES[dtype]:
            raise ValueError(f"blocks: {len(data)} bytes do not fit dtype {dtype} shape {tuple(shape)}")
        self.dtype, self.shape, self.data = dtype, tuple(int(d) for d in shape), bytes(data)

    def rows(self, r0, r1):
        """Rows [r0, r1) of a 2-D block tensor (blocks never straddle rows)."""
        rb = self.shape[1] // 32 * BLOCK_BYTES[self.dtype]
        return Blocks(self.dtype, (r1 - r0, self.shape[1]), self.data[r0 * rb:r1 * rb])


def write_nfw(path, tensors, version=3):
    """tensors: name -> np.ndarray (written F32, or F16 when its dtype is
    float16 and version >= 2) or Blocks (version 3)."""
    with open(path, "wb") as f:
        f.write(struct.pack("<IIII", MAGIC, version, len(tensors), 0))
        for name, t in tensors.items():
            if isinstance(t, Blocks):
                if version < 3:
                    raise ValueError(f"{name}: block tensors need NFW version 3")
                dtype, shape, payload = t.dtype, t.shape, t.data
            else:
                a = np.asarray(t)
                dtype = F16 if (a.dtype == np.float16 and version >= 2) else F32
                a = a.astype(np.float16 if dtype == F16 else np.float32)
                shape, payload = a.shape, np.ascontiguousarray(a).tobytes()
            nb = name.encode()
            f.write(struct.pack("<H", len(nb)) + nb + struct.pack("<B", len(shape)))
            for d in shape:
                f.write(struct.pack("<i", int(d)))
            f.write(struct.pack("<q", int(np.prod(shape)) if len(shape) else 1))
            if version >= 2:
                f.write(struct.pack("<B", dtype))
            f.write(payload)


class NfwFile:
    """An NFW file opened by the library's parser (vlrf_nfw_open)."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().vlrf_nfw_open(str(path).encode(), C.byref(h)))
        self.h = h.value

    @property
    def version(self):
        return lib().vlrf_nfw_version(self.h)

    def __len__(self):
        return lib().vlrf_nfw_count(self.h)

    def info(self, i):
        name, dtype, ndim = C.c_char_p(), C.c_int(), C.c_int()
        dims, numel, nbytes = (C.c_int32 * 8)(), C.c_int64(), C.c_int64()
        check(lib().vlrf_nfw_tensor_info(self.h, i, C.byref(name), C.byref(dtype), C.byref(ndim), dims,
                                         C.byref(numel), C.byref(nbytes)))
        return {"name": name.value.decode(), "dtype": dtype.value, "shape": tuple(dims[:ndim.value]),
                "numel": numel.value, "bytes": nbytes.value}

    def names(self):
        return [self.info(i)["name"] for i in range(len(self))]

    def find(self, name):
        return lib().vlrf_nfw_find(self.h, name.encode())

    def raw(self, i):
        n = self.info(i)["bytes"]
        buf = np.empty(n, np.uint8)
        check(lib().vlrf_nfw_read(self.h, i, buf.ctypes.data, n))
        return buf.tobytes()

    def f32(self, i):
        inf = self.info(i)
        out = np.empty(inf["numel"], np.float32)
        check(lib().vlrf_nfw_read_f32(self.h, i, out.ctypes.data, out.size))
        return out.reshape(inf["shape"])

    def close(self):
        if self.h:
            lib().vlrf_nfw_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
