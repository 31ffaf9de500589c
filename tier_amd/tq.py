""".tq quantized-base container, Python side, over the library's reader and writer.

The container (the engine reads it in tq_load / tq_of, tier.cpp:273-292; the
engine and quant.py write it, tier.cpp:2716-2744, quant.py:60-105) is a
NUL-padded text header -- ``TQB1 <hb> <n>``, ``#key value`` meta lines, one
``name type rows cols offset bytes err`` line per matrix -- followed by the
matrices at 4096-aligned offsets.  The layout, header and checks live in C
(``tiermm_tq_write`` / ``tiermm_tq_open``); this module adapts Python callers:

* ``write_tq(out, items, meta)`` and ``info(path)`` take and return what
  quant.py's functions of the same names do (item tuples with a byte source,
  the result keys ``мета``, ``матриц``, ``типы``, ``байт``, ``ошибки``), so
  tierlm.py code can call them unchanged;
* ``TqFile`` opens a base for lookups by name and row reads;
* ``check`` is the engine's ``--tq-check`` comparison of a base with its
  bf16 source model.
"""
from __future__ import annotations

import collections
import ctypes
import os

import numpy as np

from . import _L, _check, q_row_bytes

# type names of the container's lines (quant.h:26-30: the ggml ids)
TYPE_IDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11,
            "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19,
            "IQ4_NL": 20, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29, "BF16": 30, "TQ1_0": 34,
            "TQ2_0": 35, "MXFP4": 39, "NF4": 200, "FP4": 201}
TYPE_NAMES = {v: k for k, v in TYPE_IDS.items()}


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

    def entries(self) -> list[dict]:
        return [self.entry(i) for i in range(len(self))]

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
    (tiermm_tq_write: the engine's byte layout, errors with 6 decimals, "-1" without)."""
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


def _source(name: str, ty: str, rows: int, cols: int, src) -> tuple[int, np.ndarray]:
    """(type id, bytes) of one write_tq item: src is a callable returning the matrix bytes, or a
    (file, offset, size) range of another file, mapped rather than read into memory."""
    if ty not in TYPE_IDS:
        raise ValueError(f"{name}: unknown type {ty}")
    qt = TYPE_IDS[ty]
    try:
        need = q_row_bytes(qt, cols) * rows
    except Exception as e:
        raise ValueError(f"{name}: {cols} columns are not whole {ty} blocks") from e
    if callable(src):
        data = src()
        if len(data) != need:
            raise ValueError(f"{name}: {len(data)} bytes given, {ty} {rows}x{cols} takes {need}")
        return qt, np.frombuffer(data, np.uint8)
    path, offset, size = src
    if size != need:
        raise ValueError(f"{name}: the source range holds {size} bytes, {ty} {rows}x{cols} takes {need}")
    if need == 0:
        return qt, np.zeros(0, np.uint8)
    if os.path.getsize(path) < offset + size:
        raise ValueError(f"{name}: {path} ends before byte {offset + size}")
    return qt, np.memmap(path, np.uint8, mode="r", offset=offset, shape=(size,))


def write_tq(out: str, items, meta: dict) -> None:
    """quant.py:60-105's writer: items are (name, type name, rows, cols, src) with src as in
    _source; meta goes to the #key lines.  Written through out + '.part' and renamed, by
    tiermm_tq_write."""
    mats = []
    for name, ty, rows, cols, src in items:
        qt, data = _source(name, ty, rows, cols, src)
        mats.append((name, qt, rows, cols, data))
    write_tq_arrays(out, mats, meta)


def info(path: str) -> dict:
    """quant.py:314-334's summary of a base: its meta, matrix count, count per type, file size
    and the recorded per-matrix errors (those >= 0), read through tiermm_tq_open."""
    with TqFile(path) as f:
        meta, ents = f.meta(), f.entries()
    return {"мета": meta, "матриц": len(ents), "типы": dict(collections.Counter(e["type"] for e in ents)),
            "байт": os.path.getsize(path), "ошибки": {e["name"]: e["err"] for e in ents if e["err"] >= 0}}


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


def _sampled_rows(rows: int) -> list[int]:
    """The rows the engine compares: at most 48, spread evenly from the first to the last."""
    s = min(rows, 48)
    return [j * (rows - 1) // max(1, s - 1) for j in range(s)]


def _agreement(x: np.ndarray, y: np.ndarray) -> tuple[float, float, float]:
    """Squared error, squared source norm and Pearson correlation of two sample matrices
    (fp64; the correlation is 0 when either side is constant)."""
    d = y - x
    se, ss = float(np.sum(d * d)), float(np.sum(x * x))
    n = x.size
    cx, cy = x - x.sum() / n, y - y.sum() / n
    vx, vy = float(np.sum(cx * cx)), float(np.sum(cy * cy))
    cr = float(np.sum(cx * cy)) / (vx * vy) ** 0.5 if vx > 0 and vy > 0 else 0.0
    return se, ss, cr


def check(model: str, base: str, say=print) -> int:
    """tier --tq-check (tier.cpp:2749-2765): each matrix of the base (in name order) against the
    bf16 tensor of the same name in the source model, on the sampled rows: relative error and
    correlation per matrix, then the total relative error and the worst correlation.  Returns 2
    when a matrix is missing from the model or has another shape, or correlates below 0.5 (a
    base of another model), else 0.  The printed lines keep the engine's wording; quant.py
    (quant.py:337-358) parses the last one."""
    from . import dequant_host
    tab, data0 = _safetensors_index(model)
    with TqFile(base) as f, open(model, "rb") as src:
        ents = sorted(f.entries(), key=lambda e: e["name"].encode())
        total_se = total_ss = 0.0
        worst, worst_name, bad = 1.0, "", 0
        for k, e in enumerate(ents, 1):
            head = f"Сверка {k}/{len(ents)} {e['name']}"
            t = tab.get(e["name"])
            if (t is None or t[3] - t[2] != e["rows"] * e["cols"] * 2
                    or (len(t[1]) >= 2 and t[1][-1] != e["cols"])):
                say(f"{head}: в модели нет такой матрицы или у неё другая форма.")
                bad += 1
                continue
            rows = _sampled_rows(e["rows"])
            i = f.find(e["name"])
            xs, ys = [], []
            for r in rows:
                src.seek(data0 + t[2] + r * e["cols"] * 2)
                xs.append(np.frombuffer(src.read(e["cols"] * 2), np.uint16))
                ys.append(dequant_host(f.read_rows(i, r, 1), e["qtype"], e["cols"])[0])
            x = (np.stack(xs).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            se, ss, cr = _agreement(x, np.stack(ys).astype(np.float64))
            total_se += se
            total_ss += ss
            if cr < worst:
                worst, worst_name = cr, e["name"]
            bad += cr < 0.5
            rel = (se / ss) ** 0.5 if ss > 0 else 0.0
            say(f"{head} {e['type']}, ошибка {100 * rel:.2f}%, корреляция {cr:.4f}")
    total = 100 * (total_se / total_ss) ** 0.5 if total_ss > 0 else 0.0
    say(f"Итог: ошибка весов {total:.2f}%, худшая корреляция {worst:.4f} ({worst_name})"
        f"{', обнаружены матрицы от другой модели' if bad else ''}")
    return 2 if bad else 0
