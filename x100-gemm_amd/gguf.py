"""GGUF checkpoints on the GPU path: a reader over libx100hip's native parser (include/x100_gguf.h),
a writer for GGUF v3 files, and the listing of bench/gguf_dump.c.

Reader (the reference's gguf_open / gguf_find, qwen_moe.c:110-154):

    with gguf.GGUF("model.gguf") as g:
        p = g.qwen3moe()                       # block_count, embd, n_exp, ... (qwen_moe.c:129-151)
        t = g.find("blk.0.ffn_gate_exps.weight")
        g.upload(t, dev_ptr, stream)           # raw GGUF blocks -> device (moe_layer_hip eats them)
        g.pack_rows(t, 0, n, packed, stream)   # rows -> qgemv_hip layout

The file is mapped, not read: tensor bytes go from the page cache to the device.  Nothing here
dequantizes; the kernels consume ggml blocks.

Writer: write(path, kv, tensors) with kv = [(key, type, value)] (arrays as
(ARRAY, (elem_type, values))) and tensors = [(name, ggml_type, dims_ggml_order, raw_bytes)].
"""
import ctypes
import struct
import sys

import numpy as np

import x100hip

# metadata value types (GGUF spec; x100_gguf.h)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
               U64: "<Q", I64: "<q", F64: "<d"}

# ggml type ids (bench/gguf_dump.c:12-14)
F32_T, F16_T, Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 3, 8, 11, 12, 13, 14, 15


class Tensor(ctypes.Structure):
    """x100_gguf_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("n_elems", ctypes.c_uint64),
                ("n_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    @property
    def shape(self):
        """dims in ggml order (contiguous dimension first)."""
        return tuple(int(self.dims[d]) for d in range(self.n_dims))

    def array(self):
        """The tensor's bytes as a read-only uint8 view of the mapping (valid while the file is
        open)."""
        if not self.data or not self.n_bytes:
            raise ValueError("tensor %s has no known byte size" % self.name.decode())
        buf = (ctypes.c_uint8 * self.n_bytes).from_address(self.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a


class Qwen3MoeParams(ctypes.Structure):
    """x100_gguf_qwen3moe."""
    _fields_ = [(n, ctypes.c_int) for n in ("block_count", "embd", "ffn", "n_head", "n_head_kv", "head_dim",
                                            "vocab", "n_exp", "n_act", "moe_ffn")] + \
               [("rope_base", ctypes.c_float), ("n_tokens", ctypes.c_int)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class GGUF:
    """A mapped GGUF file (x100_gguf_open)."""

    def __init__(self, path):
        self._L = x100hip.lib()
        h = ctypes.c_void_p()
        x100hip._check("x100_gguf_open", self._L.x100_gguf_open(path.encode() if isinstance(path, str) else path,
                                                                 ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            self._L.x100_gguf_close(self._h)
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

    # ---- header ---------------------------------------------------------------------------
    @property
    def version(self):
        return self._L.x100_gguf_version(self._h)

    @property
    def n_tensors(self):
        return self._L.x100_gguf_n_tensors(self._h)

    @property
    def n_kv(self):
        return self._L.x100_gguf_n_kv(self._h)

    @property
    def alignment(self):
        return self._L.x100_gguf_alignment(self._h)

    @property
    def data_offset(self):
        return self._L.x100_gguf_data_offset(self._h)

    # ---- tensors --------------------------------------------------------------------------
    def tensor(self, i):
        t = Tensor()
        x100hip._check("x100_gguf_tensor_at", self._L.x100_gguf_tensor_at(self._h, i, ctypes.byref(t)))
        return t

    def tensors(self):
        return [self.tensor(i) for i in range(self.n_tensors)]

    def find(self, name):
        t = Tensor()
        x100hip._check("x100_gguf_find", self._L.x100_gguf_find(self._h, name.encode(), ctypes.byref(t)))
        return t

    def has(self, name):
        t = Tensor()
        return self._L.x100_gguf_find(self._h, name.encode(), ctypes.byref(t)) == x100hip.X100_OK

    def upload(self, t, dst, stream=None, byte0=0, n=None):
        n = t.n_bytes - byte0 if n is None else n
        return x100hip._check("x100_gguf_upload", self._L.x100_gguf_upload(self._h, ctypes.byref(t), byte0, n,
                                                                          dst, stream))

    def pack_rows(self, t, row0, n_rows, w_packed, stream=None):
        return x100hip._check("x100_gguf_pack_rows", self._L.x100_gguf_pack_rows(
            self._h, ctypes.byref(t), row0, n_rows, w_packed, stream))

    # ---- metadata -------------------------------------------------------------------------
    def kv_at(self, i):
        key, typ, et, cnt = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        x100hip._check("x100_gguf_kv_at", self._L.x100_gguf_kv_at(self._h, i, ctypes.byref(key), ctypes.byref(typ),
                                                                  ctypes.byref(et), ctypes.byref(cnt)))
        return key.value, typ.value, et.value, cnt.value

    def keys(self):
        return [self.kv_at(i)[0].decode() for i in range(self.n_kv)]

    def get_int(self, key):
        v = ctypes.c_int64()
        x100hip._check("x100_gguf_get_int", self._L.x100_gguf_get_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_float(self, key):
        v = ctypes.c_double()
        x100hip._check("x100_gguf_get_float", self._L.x100_gguf_get_float(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_bytes(self, key):
        s, n = ctypes.c_void_p(), ctypes.c_uint64()
        x100hip._check("x100_gguf_get_str", self._L.x100_gguf_get_str(self._h, key.encode(), ctypes.byref(s),
                                                                      ctypes.byref(n)))
        return ctypes.string_at(s.value, n.value) if n.value else b""

    def get_str(self, key):
        return self.get_bytes(key).decode("utf-8", "replace")

    def get_arr_str(self, key, j):
        s, n = ctypes.c_void_p(), ctypes.c_uint64()
        x100hip._check("x100_gguf_get_arr_str", self._L.x100_gguf_get_arr_str(
            self._h, key.encode(), j, ctypes.byref(s), ctypes.byref(n)))
        return ctypes.string_at(s.value, n.value) if n.value else b""

    def qwen3moe(self):
        p = Qwen3MoeParams()
        x100hip._check("x100_gguf_qwen3moe_params", self._L.x100_gguf_qwen3moe_params(self._h, ctypes.byref(p)))
        return p.as_dict()


def type_name(t):
    return x100hip.lib().x100_gguf_type_name(t).decode()


# ------------------------------------------------------------------------------------------------
# bench/gguf_dump.c listing
# ------------------------------------------------------------------------------------------------
_SHOWN = ("architecture", "expert", "block_count", "head_count", "embedding_length", "feed_forward",
          "context_length", "vocab", "rope", "tokenizer.ggml.model", "attention.key_length",
          "attention.value_length")


def _c255(b):
    """A GGUF string as the reference tool holds it: at most 255 bytes, cut at a NUL."""
    b = b[:255]
    return b.split(b"\0", 1)[0]


def dump(path, grep=None):
    """The text bench/gguf_dump.c prints for `gguf_dump path [grep]` (bytes): the header line, the
    selected keys (gguf_dump.c:60-66, printval :33-42), then up to 40 tensors (all that match
    `grep` when it is given) with type name, dims and offset (:68-80)."""
    out = []
    with GGUF(path) as g:
        out.append(b"magic=GGUF ver=%d  n_tensors=%d  n_kv=%d\n" % (g.version, g.n_tensors, g.n_kv))
        for i in range(g.n_kv):
            key, typ, et, cnt = g.kv_at(i)
            k = _c255(key)
            if not any(s.encode() in k for s in _SHOWN):
                continue
            ks = k.decode("latin-1")
            if typ == STRING:
                val = _c255(g.get_bytes(ks))
            elif typ in (U32, U64):
                val = b"%d" % g.get_int(ks)
            elif typ in (I32, I64):
                val = b"%d" % g.get_int(ks)
            elif typ == F32:
                val = (b"%g" % g.get_float(ks))
            elif typ == ARRAY:
                val = b"[array type=%d n=%d]" % (et, cnt)
            else:
                val = b"<t%d>" % typ
            out.append(b"  %-45s = %s\n" % (k, val))
        out.append(b"--- tensors (name  type  dims  offset) ---\n")
        shown = 0
        gb = grep.encode() if isinstance(grep, str) else grep
        for t in g.tensors():
            name = _c255(t.name)
            if gb is None or gb in name:
                if shown < 40 or gb is not None:
                    dims = b"x".join(b"%d" % d for d in t.shape)
                    out.append(b"  %-30s %-6s [%s]  @%d\n" % (name, type_name(t.type).encode(), dims, t.offset))
                shown += 1
        out.append(b"(%d tensors listed of %d)\n" % (shown, g.n_tensors))
    return b"".join(out)


# ------------------------------------------------------------------------------------------------
# writer
# ------------------------------------------------------------------------------------------------
def _str(b):
    b = b.encode() if isinstance(b, str) else bytes(b)
    return struct.pack("<Q", len(b)) + b


def _value(typ, v):
    if typ in _SCALAR_FMT:
        return struct.pack(_SCALAR_FMT[typ], v)
    if typ == STRING:
        return _str(v)
    if typ == ARRAY:
        et, vals = v
        return struct.pack("<IQ", et, len(vals)) + b"".join(_value(et, x) for x in vals)
    raise ValueError("metadata type %r" % typ)


def write(path, kv, tensors, alignment=32, version=3):
    """Write a GGUF file.  kv: [(key, type, value)]; tensors: [(name, ggml_type, dims, bytes)] with
    dims in ggml order.  Tensor data is laid out in list order, each at a multiple of
    `alignment` from the start of the data section.  Returns the list of data offsets."""
    head = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(kv))]
    for key, typ, v in kv:
        head.append(_str(key) + struct.pack("<I", typ) + _value(typ, v))
    offs, off = [], 0
    for name, gt, dims, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        head.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                    struct.pack("<IQ", gt, off))
        off += len(data)
    blob = b"".join(head)
    pad = (-len(blob)) % alignment
    with open(path, "wb") as f:
        f.write(blob + b"\0" * pad)
        pos = 0
        for (name, gt, dims, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(bytes(data))
            pos = o + len(data)
    return offs


def main(argv):
    """gguf_dump file.gguf [namegrep] -- the listing of bench/gguf_dump.c."""
    if len(argv) < 2:
        print("usage: %s file.gguf [namegrep]" % argv[0])
        return 1
    try:
        sys.stdout.buffer.write(dump(argv[1], argv[2] if len(argv) > 2 else None))
    except x100hip.X100Error as e:
        print(e)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
