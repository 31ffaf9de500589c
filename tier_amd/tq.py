""".tq quantized-base container: the Python side of tierlm's format.

``write_tq`` and ``info`` keep the interface of quant.py's writer and reader
(quant.py:60-105 and 314-334: the same item tuples, the same header bytes, the
same result keys) so tierlm.py code can call them unchanged; ``TqFile`` reads
a base through the library's parser (tiermm_tq_*, the checks of tq_load,
tier.cpp:273-292) and hands rows to device memory.

Format: a NUL-padded text header of hb bytes -- ``TQB1 <hb> <n>``, ``#key
value`` meta lines, one ``name type rows cols offset bytes err`` line per
matrix -- with hb = ceil((n*200 + 4096) / 4096) * 4096, then the matrices at
4096-aligned offsets.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

from . import _L, _check, TYPE_NAMES, q_info

# block geometry by type name (quant.h:26-30)
_TYPES = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
          "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


def _geometry(ty: str):
    if ty not in _TYPES:
        raise ValueError(f"unknown type {ty}")
    return q_info(_TYPES[ty])


def write_tq(out: str, items, meta: dict) -> None:
    """quant.py:60-105: items are (name, type, rows, cols, src); src is a callable returning
    the matrix bytes or a (file, offset, size) triple to copy from.  Written through
    ``out + '.part'`` and renamed."""
    items = list(items)
    hb = (len(items) * 200 + 4096 + 4095) // 4096 * 4096
    off, lay = hb, []
    for nm, ty, rows, cols, src in items:
        b, by = _geometry(ty)
        if cols % b:
            raise ValueError(f"{nm}: {cols} columns are not whole {ty} blocks of {b}")
        size = cols // b * by * rows
        lay.append((nm, ty, rows, cols, off, size, src))
        off += (size + 4095) // 4096 * 4096
    tmp = out + ".part"
    with open(tmp, "wb") as f:
        f.truncate(off)
        for nm, ty, rows, cols, o, size, src in lay:
            f.seek(o)
            if callable(src):
                data = src()
                if len(data) != size:
                    raise ValueError(f"{nm}: {len(data)} bytes given, {size} needed")
                f.write(data)
            else:
                fn, so, sn = src
                if sn != size:
                    raise ValueError(f"{nm}: the source holds {sn} bytes, {ty} {rows}x{cols} needs {size}")
                with open(fn, "rb") as g:
                    g.seek(so)
                    left = size
                    while left:
                        chunk = g.read(min(left, 64 << 20))
                        if not chunk:
                            raise ValueError(f"{nm}: the source ends early")
                        f.write(chunk)
                        left -= len(chunk)
        head = f"TQB1 {hb} {len(lay)}\n" + "".join(f"#{k} {v}\n" for k, v in meta.items())
        head += "".join(f"{nm} {ty} {rows} {cols} {o} {size} -1\n" for nm, ty, rows, cols, o, size, _ in lay)
        raw = head.encode()
        if len(raw) >= hb:
            raise ValueError("the header does not fit its reserved space")
        f.seek(0)
        f.write(raw.ljust(hb, b"\0"))
    os.replace(tmp, out)


def info(path: str) -> dict:
    """quant.py:314-334: meta, matrix count, types, file size and the per-matrix errors."""
    with open(path, "rb") as f:
        first = f.readline().decode()
        m = re.match(r"^TQB1 (\d+) (\d+)", first)
        if not m:
            raise ValueError(f"{path} is not a .tq file")
        f.seek(0)
        h = f.read(int(m.group(1))).split(b"\0", 1)[0].decode()
    meta, mats, types, errs = {}, 0, {}, {}
    for line in h.splitlines()[1:]:
        if line.startswith("#"):
            k, _, v = line[1:].partition(" ")
            meta[k] = v
            continue
        p = line.split()
        if len(p) >= 6:
            mats += 1
            types[p[1]] = types.get(p[1], 0) + 1
            if len(p) >= 7 and float(p[6]) >= 0:
                errs[p[0]] = float(p[6])
    return {"мета": meta, "матриц": mats, "типы": types, "байт": os.path.getsize(path), "ошибки": errs}


class TqFile:
    """A parsed .tq base (tiermm_tq_open): matrix lookup by name and row reads."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(_L.tiermm_tq_open(path.encode(), ctypes.byref(h)))
        self._h = h
        self.path = path

    def close(self) -> None:
        if self._h:
            _L.tiermm_tq_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return _L.tiermm_tq_count(self._h)

    def find(self, name: str) -> int:
        return _L.tiermm_tq_find(self._h, name.encode())

    def entry(self, i: int) -> dict:
        nm = ctypes.c_char_p()
        qt, rows, cols = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        off, size, rb, err = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_size_t(), ctypes.c_double()
        _check(_L.tiermm_tq_info(self._h, i, ctypes.byref(nm), ctypes.byref(qt), ctypes.byref(rows), ctypes.byref(cols),
                                 ctypes.byref(off), ctypes.byref(size), ctypes.byref(rb), ctypes.byref(err)))
        return {"name": nm.value.decode(), "qtype": qt.value, "type": TYPE_NAMES.get(qt.value, str(qt.value)),
                "rows": rows.value, "cols": cols.value, "offset": off.value, "bytes": size.value, "rb": rb.value,
                "err": err.value}

    def meta(self) -> dict:
        out = {}
        for i in range(_L.tiermm_tq_meta_count(self._h)):
            k, v = ctypes.c_char_p(), ctypes.c_char_p()
            _check(_L.tiermm_tq_meta(self._h, i, ctypes.byref(k), ctypes.byref(v)))
            out[k.value.decode()] = v.value.decode()
        return out

    def read_rows(self, i: int, r0: int = 0, nrows: int | None = None) -> np.ndarray:
        e = self.entry(i)
        n = e["rows"] - r0 if nrows is None else nrows
        buf = np.empty((n, e["rb"]), np.uint8)
        _check(_L.tiermm_tq_read_rows(self._h, i, r0, n, buf.ctypes.data_as(ctypes.c_void_p)))
        return buf


def write_tq_arrays(out: str, mats, meta: dict | None = None, errs=None) -> None:
    """Write (name, qtype id, rows, cols, uint8 array) matrices with the library writer
    (tiermm_tq_write: the engine's byte layout, errors with 6 decimals)."""
    mats = list(mats)
    n = len(mats)
    meta = meta or {}
    arrs = [np.ascontiguousarray(a, np.uint8) for *_, a in mats]
    names = (ctypes.c_char_p * n)(*[m[0].encode() for m in mats])
    qt = (ctypes.c_int * n)(*[m[1] for m in mats])
    rows = (ctypes.c_int * n)(*[m[2] for m in mats])
    cols = (ctypes.c_int * n)(*[m[3] for m in mats])
    data = (ctypes.c_void_p * n)(*[a.ctypes.data for a in arrs])
    e = (ctypes.c_double * n)(*errs) if errs is not None else None
    keys = (ctypes.c_char_p * max(1, len(meta)))(*[k.encode() for k in meta])
    vals = (ctypes.c_char_p * max(1, len(meta)))(*[str(v).encode() for v in meta.values()])
    _check(_L.tiermm_tq_write(out.encode(), n, names, qt, rows, cols, data, e, len(meta), keys, vals))
