"""Writes tests/golden/q4k_tiny.npz and tests/golden/q6k_tiny.npz from the reference's own test
fixtures (data only): tests/fixtures/tiny.gguf's Q4_K tensor "q4_k" and Q6_K tensor "q6_k" (their
raw GGUF blocks) and tests/fixtures/tiny.q4_k.f32 / tiny.q6_k.f32 (the same tensors dequantized
by the reference, the files its tests compare against). Run in a container that holds the
reference tree:

    python tests/golden/make_quant_fixtures.py [/path/to/reference]

The GGUF container is parsed here (header, key/value pairs, tensor infos, aligned data section);
no reference code is imported or run.
"""
from __future__ import annotations

import struct
import sys
from pathlib import Path

import numpy as np

_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
            11: "<q", 12: "<d"}


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.o = data, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.d, self.o)[0]
        self.o += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = self.d[self.o:self.o + n].decode()
        self.o += n
        return s

    def value(self, t):
        if t in _SCALARS:
            return self.take(_SCALARS[t])
        if t == 8:
            return self.string()
        if t == 9:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"GGUF value type {t}")


def gguf_tensors(path: Path):
    """{name: (ggml type, dims, raw bytes of the tensor's data)} of a GGUF v2/v3 file."""
    data = path.read_bytes()
    r = _Reader(data)
    if data[:4] != b"GGUF":
        raise ValueError("not a GGUF file")
    r.o = 4
    version, n_tensors, n_kv = r.take("<I"), r.take("<Q"), r.take("<Q")
    if version < 2:
        raise ValueError(f"GGUF version {version}")
    kv = {}
    for _ in range(n_kv):
        key = r.string()
        kv[key] = r.value(r.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        dims = [r.take("<Q") for _ in range(r.take("<I"))]
        infos.append((name, dims, r.take("<I"), r.take("<Q")))
    align = int(kv.get("general.alignment", 32))
    base = (r.o + align - 1) // align * align
    sizes = {12: (256, 144), 14: (256, 210), 0: (1, 4), 1: (1, 2)}
    out = {}
    for name, dims, t, off in infos:
        n = int(np.prod(dims))
        per, nbytes = sizes.get(t, (None, None))
        if per is None:
            continue
        out[name] = (t, dims, data[base + off: base + off + n // per * nbytes])
    return out


def main(ref: Path) -> None:
    fx = ref / "tests" / "fixtures"
    tensors = gguf_tensors(fx / "tiny.gguf")
    for name, ggml_type, block_bytes in (("q4_k", 12, 144), ("q6_k", 14, 210)):
        t, dims, raw = tensors[name]
        assert t == ggml_type, (name, t)
        expect = np.fromfile(fx / f"tiny.{name}.f32", dtype="<f4")
        k, n = int(dims[0]), int(np.prod(dims[1:]))
        assert expect.size == k * n and len(raw) == k * n // 256 * block_bytes
        out = Path(__file__).resolve().parent / f"{name.replace('_', '')}_tiny.npz"
        np.savez_compressed(out, blocks=np.frombuffer(raw, np.uint8), dequant=expect,
                            k=np.int64(k), n=np.int64(n))
        print(f"{out}: K={k} N={n}, {len(raw)} bytes of {name} blocks")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
