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

from . import _L, _check, q_info

# block geometry by type name (quant.h:26-30)
_TYPES = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
          "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23, "TQ1_0": 34, "TQ2_0": 35,
          "MXFP4": 39, "NF4": 200, "FP4": 201}


_NAMES = {v: k for k, v in _TYPES.items()}


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
        return {"name": nm.value.decode(), "qtype": qt.value, "type": _NAMES.get(qt.value, str(qt.value)),
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


def _safetensors_index(path: str) -> tuple[dict, int]:
    """Tensor table of a safetensors file: {name: (dtype, shape, begin, end)}, data start."""
    import json
    import struct
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        head = json.loads(f.read(n))
    tab = {k: (v["dtype"], tuple(v["shape"]), v["data_offsets"][0], v["data_offsets"][1])
           for k, v in head.items() if k != "__metadata__"}
    return tab, 8 + n


def check(model: str, base: str, say=print) -> int:
    """tier --tq-check (tier.cpp:2749-2765): for every matrix of the base (by name order),
    up to 48 rows spread evenly over the matrix are dequantized (q_val) and compared with the
    bf16 source tensor: relative error and correlation per matrix, then the total error and
    the worst correlation.  Returns 2 when a matrix is missing from the model, has another
    shape, or correlates below 0.5 (a base of another model), else 0.  The last line keeps
    the engine's wording, which quant.py's check (quant.py:337-358) parses."""
    from . import dequant_host
    tab, data0 = _safetensors_index(model)
    SE = SS = 0.0
    worst, wname, bad = 1.0, "", 0
    with TqFile(base) as f, open(model, "rb") as src:
        entries = sorted((f.entry(i) for i in range(len(f))), key=lambda e: e["name"].encode())
        for k, e in enumerate(entries, 1):
            t = tab.get(e["name"])
            cols_ok = t is not None and (len(t[1]) < 2 or t[1][-1] == e["cols"])
            if t is None or t[3] - t[2] != e["rows"] * e["cols"] * 2 or not cols_ok:
                say(f"Сверка {k}/{len(entries)} {e['name']}: в модели нет такой матрицы или у неё другая форма.")
                bad += 1
                continue
            S = min(e["rows"], 48)
            rows = [j * (e["rows"] - 1) // max(1, S - 1) for j in range(S)]
            se = ss = sx = sy = sxy = sxx = syy = 0.0
            n = 0
            i = f.find(e["name"])
            for r in rows:
                src.seek(data0 + t[2] + r * e["cols"] * 2)
                raw = np.frombuffer(src.read(e["cols"] * 2), np.uint16)
                x = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
                y = dequant_host(f.read_rows(i, r, 1), e["qtype"], e["cols"])[0].astype(np.float64)
                d = y - x
                se += float(d @ d); ss += float(x @ x); sx += float(x.sum()); sy += float(y.sum())
                sxy += float(x @ y); sxx += float(x @ x); syy += float(y @ y)
                n += x.size
            cov, vx, vy = sxy - sx * sy / n, sxx - sx * sx / n, syy - sy * sy / n
            cr = cov / (vx * vy) ** 0.5 if vx > 0 and vy > 0 else 0.0
            er = (se / ss) ** 0.5 if ss > 0 else 0.0
            SE += se
            SS += ss
            if cr < worst:
                worst, wname = cr, e["name"]
            if cr < 0.5:
                bad += 1
            say(f"Сверка {k}/{len(entries)} {e['name']} {e['type']}, ошибка {100 * er:.2f}%, "
                f"корреляция {cr:.4f}")
    total = 100 * (SE / SS) ** 0.5 if SS > 0 else 0.0
    say(f"Итог: ошибка весов {total:.2f}%, худшая корреляция {worst:.4f} ({wname})"
        f"{', обнаружены матрицы от другой модели' if bad else ''}")
    return 2 if bad else 0
