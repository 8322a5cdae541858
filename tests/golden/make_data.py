"""Write the small data files the runtime fixtures read (tests/golden/data/): a CSV table with a
header and numbers in several spellings, a text file read as bytes, gzip'ed and plain IDX files,
a .npy file of every element kind the language reads, and a .safetensors file. Deterministic: the
committed files are what this script writes.

    python tests/golden/make_data.py
"""
import gzip
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "data")


def idx(dtype_code: int, shape, payload: bytes) -> bytes:
    head = struct.pack(">BBBB", 0, 0, dtype_code, len(shape)) + b"".join(struct.pack(">I", d) for d in shape)
    return head + payload


def main() -> None:
    os.makedirs(OUT, exist_ok=True)
    with open(os.path.join(OUT, "table.csv"), "w") as f:
        f.write("alpha,beta,gamma\n")
        f.write("1.5,-2,.25\n")
        f.write("3e2,+4.,-0.125\n")
        f.write(" 7 ,1E-3,-6.5e+1\n")
        f.write("0.1,2.5e0,12\n")
    with open(os.path.join(OUT, "note.txt"), "wb") as f:
        f.write(b"MI355X: 8 XCDs\n\x00\xff")
    rng = np.random.default_rng(7)
    pixels = rng.integers(0, 256, size=(3, 4, 5), dtype=np.uint8)
    with gzip.GzipFile(os.path.join(OUT, "tiles-idx3-ubyte.gz"), "wb", mtime=0) as f:
        f.write(idx(8, pixels.shape, pixels.tobytes()))
    with open(os.path.join(OUT, "marks-idx1-ubyte"), "wb") as f:
        f.write(idx(8, (6,), bytes([0, 9, 255, 3, 128, 1])))
    arrays = {
        "k_f4": np.array([[1.5, -2.25, 3.0e-5], [7.0, -0.0, 1.0e7]], np.float32),
        "k_f8": np.array([0.1, -1.0 / 3.0, 1.0e-40, 6.02214076e23], np.float64),
        "k_f2": np.array([1.0, -0.5, 6.0e-8, 65504.0, np.inf, -np.inf, 0.333], np.float16),
        "k_i4": np.array([-7, 0, 2147483647], np.int32),
        "k_i8": np.array([5, -3, (1 << 33) + 9], np.int64),
        "k_u1": np.array([0, 1, 200, 255], np.uint8),
        "k_i1": np.array([-128, -1, 0, 127], np.int8),
        "k_u2": np.array([0, 65535, 300], np.uint16),
        "k_i2": np.array([-32768, 12, 32767], np.int16),
        "k_b1": np.array([True, False, True], np.bool_),
    }
    for name, a in arrays.items():
        np.save(os.path.join(OUT, f"{name}.npy"), a)
    # a .safetensors file: 8-byte little-endian header length, the JSON header, then the data
    tensors = {"layer.w": np.arange(6, dtype=np.float32).reshape(2, 3) / 4 - 0.5,
               "layer.half": np.array([0.5, -2.0, 1024.0], np.float16),
               "layer.ids": np.array([[3, -4], [1 << 20, 9]], np.int64)}
    codes = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int64): "I64"}
    header, blobs, at = {}, [], 0
    for name, a in tensors.items():
        raw = a.tobytes()
        header[name] = {"dtype": codes[a.dtype], "shape": list(a.shape), "data_offsets": [at, at + len(raw)]}
        blobs.append(raw)
        at += len(raw)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)
    with open(os.path.join(OUT, "layer.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))


if __name__ == "__main__":
    main()
