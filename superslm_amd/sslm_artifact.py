""".sslm v2 artifact writer and seeded synthetic model generator.

Format restated from the reference's normative spec (docs/sslm_format.md:47-118 header and
section table, :178-240 WGT1/BIA1/ROP1/WSC1 tensor manifests, :242-290 KVC1 keyed constants,
:292-327 CFG1, :340-365 SIL1).  Names follow include/superslm/layer_marshal.h:141-330 and
src/sslm_abi.cpp:609-676 (embed / final_norm.gain / lm_head, site constants).

The generator draws every weight from a seeded numpy PCG64 stream and derives every composition
constant from one consistent "real value per code" model, so a synthetic stack stays inside the
reference's load-time value gate (src/model.cpp:940-1180) and inside the runtime domains (funnel
D' <= 2^31, i-exp constants, SiLU scale range) for whole forwards.  There is no network and no
checkpoint: synthetic artifacts are how every BASELINE configuration gets a real .sslm.
"""
from __future__ import annotations

import hashlib
import math
import struct
from dataclasses import dataclass, field

import numpy as np

# ---- section / dtype enums (docs/sslm_format.md:100-139) ----
SEC_CONFIG = 0
SEC_PROVENANCE = 1
SEC_WEIGHTS = 2
SEC_BIASES = 3
SEC_ROPE = 4
SEC_WEIGHT_SCALES = 6
SEC_COMPOSITION = 7
SEC_KV_LANDING_SCALES = 8
SEC_KV_LANDING_RECIPROCALS = 9
SEC_SIGMOID_LUT = 12
SEC_DELTA_FOLD = 40
SEC_U_FOLD = 41
SEC_DAMPED_GREEDY = 42
SEC_SCHEMA_MASKS = 30

DT_RAW, DT_I8, DT_I32, DT_I64 = 0, 1, 2, 3
_DT_SIZE = {DT_RAW: 1, DT_I8: 1, DT_I32: 4, DT_I64: 8}

HEADER_BYTES = 64
SECTION_DESC_BYTES = 40
HASH_OFFSET = 32

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def write_container(sections, flags: int = 0) -> bytes:
    """sections: list of (type, dtype, payload, alignment) with payload bytes or a Manifest.
    Returns the whole file with the SHA-256 integrity field filled (docs/sslm_format.md:26-32)."""
    return bytes(write_container_array(sections, flags))


def with_flags(image: bytes, flags: int) -> bytes:
    """The container `image` with header flags `flags` (bit 0: Option-G fused K landing, bit 1:
    damped-greedy constants; src/artifact.cpp:254-270, :511-518) and its integrity SHA-256
    recomputed (over the file with the hash field zeroed)."""
    b = bytearray(image)
    struct.pack_into("<I", b, 16, flags)
    b[32:64] = hashlib.sha256(bytes(b[:32]) + bytes(32) + bytes(b[64:])).digest()
    return bytes(b)


def scm1(vocab: int, schemas) -> bytes:
    """SchemaMasks section (include/superslm/schema_masks.h): header "SCM1", version 1, count,
    vocab, name-blob length, 0; 56-byte descriptors (name offset/length, state, accepting and
    transition counts, 0, then u64 offsets of the mask pages, state offsets, accepting set and
    transitions, relative to the section); the name blob; the blocks.  `schemas`: (name,
    {state: {token: next}}, accepting) with states 0..n-1; mask bits follow the transitions."""
    page = (vocab + 7) // 8
    names = b"".join(n.encode() for n, _, _ in schemas)
    head = 24 + 56 * len(schemas) + len(names)
    cursor = (head + 7) // 8 * 8
    descs, blocks, name_off = [], [], 0
    for name, table, accepting in schemas:
        n = max(table) + 1 if table else 1
        n = max(n, max((max(r.values()) for r in table.values() if r), default=0) + 1,
                max(accepting, default=0) + 1)
        pages = bytearray(n * page)
        offsets, trans = [0], []
        for st in range(n):
            for tok in sorted(table.get(st, {})):
                pages[st * page + tok // 8] |= 1 << (tok % 8)
                trans.append(struct.pack("<II", tok, table[st][tok]))
            offsets.append(len(trans))
        parts = [bytes(pages), struct.pack(f"<{n + 1}I", *offsets),
                 struct.pack(f"<{len(accepting)}I", *sorted(accepting)), b"".join(trans)]
        offs = []
        for part in parts:
            offs.append(cursor)
            blocks.append((cursor, part))
            cursor = (cursor + len(part) + 7) // 8 * 8
        descs.append(struct.pack("<6I4Q", name_off, len(name.encode()), n, len(accepting), len(trans), 0, *offs))
        name_off += len(name.encode())
    out = bytearray(cursor)
    out[:24] = struct.pack("<4s5I", b"SCM1", 1, len(schemas), vocab, len(names), 0)
    out[24:24 + 56 * len(schemas)] = b"".join(descs)
    out[24 + 56 * len(schemas):head] = names
    for off, part in blocks:
        out[off:off + len(part)] = part
    return bytes(out)


def write_container_array(sections, flags: int = 0) -> np.ndarray:
    """Same as write_container, returning the file image as a uint8 array (no extra copy)."""
    count = len(sections)
    table_end = HEADER_BYTES + count * SECTION_DESC_BYTES
    offsets = []
    cursor = table_end
    for _t, _d, payload, align in sections:
        cursor = _align(cursor, align)
        offsets.append(cursor)
        cursor += payload.size if isinstance(payload, Manifest) else len(payload)
    total = cursor
    buf = np.zeros(total, dtype=np.uint8)
    buf[:HEADER_BYTES] = np.frombuffer(
        struct.pack("<4sIIIIIQ", b"SSLM", 2, HEADER_BYTES, count, flags, 0, total).ljust(HEADER_BYTES, b"\0"),
        dtype=np.uint8)
    for i, ((typ, dt, payload, align), off) in enumerate(zip(sections, offsets)):
        size = payload.size if isinstance(payload, Manifest) else len(payload)
        if size % _DT_SIZE[dt]:
            raise ValueError(f"section {typ}: {size} bytes is not a multiple of dtype size")
        row = struct.pack("<IIQQQII", typ, dt, off, size, size // _DT_SIZE[dt], align, 0)
        base = HEADER_BYTES + i * SECTION_DESC_BYTES
        buf[base:base + SECTION_DESC_BYTES] = np.frombuffer(row, dtype=np.uint8)
        if isinstance(payload, Manifest):
            payload.write_into(buf[off:off + size])
        else:
            buf[off:off + size] = np.frombuffer(payload, dtype=np.uint8)
    digest = hashlib.sha256(memoryview(buf)).digest()  # hash field is still zero here
    buf[HASH_OFFSET:HASH_OFFSET + 32] = np.frombuffer(digest, dtype=np.uint8)
    return buf


class RandI8:
    """A weight tensor not yet drawn: uniform int8 codes in [-127, 127] written straight into the
    artifact image (one pass over fresh memory for multi-GB models)."""

    def __init__(self, shape):
        self.shape = tuple(shape)
        self.ndim = len(self.shape)
        self.size = int(np.prod(self.shape))
        self.nbytes = self.size
        self.dtype = np.dtype(np.int8)


class Manifest:
    """A WGT1/BIA1/ROP1/WSC1/DFS1/UFS1 tensor manifest (docs/sslm_format.md:200-238) laid out
    lazily: `size` is known up front and `write_into` fills a caller buffer, so multi-GB weight
    sections are copied exactly once, into the final file image."""

    def __init__(self, magic: bytes, elem_size: int, tensors):
        self.magic = magic
        self.elem = elem_size
        self.tensors = [(n, a if isinstance(a, RandI8) else np.ascontiguousarray(a)) for n, a in tensors]
        self.rng = None
        names = [n.encode() for n, _ in self.tensors]
        self.name_blob = b"".join(names)
        count = len(self.tensors)
        self.head = 16 + 48 * count
        cursor = _align(self.head + len(self.name_blob), elem_size)
        descs = bytearray()
        self.offsets = []
        name_off = 0
        for (name, a), nb in zip(self.tensors, names):
            if a.dtype.itemsize != elem_size:
                raise ValueError(f"{name}: element size {a.dtype.itemsize} != {elem_size}")
            shape = list(a.shape) + [0] * (4 - a.ndim)
            cursor = _align(cursor, elem_size)
            descs += struct.pack("<III4IQQI", name_off, len(nb), a.ndim, *shape, cursor, a.size, 0)
            self.offsets.append(cursor)
            cursor += a.nbytes
            name_off += len(nb)
        self.descs = bytes(descs)
        self.size = _align(cursor, 8)

    def write_into(self, out: np.ndarray):
        out[:self.size] = 0
        out[:16] = np.frombuffer(struct.pack("<4sIII", self.magic, 1, len(self.tensors), len(self.name_blob)),
                                 dtype=np.uint8)
        out[16:16 + len(self.descs)] = np.frombuffer(self.descs, dtype=np.uint8)
        if self.name_blob:
            out[self.head:self.head + len(self.name_blob)] = np.frombuffer(self.name_blob, dtype=np.uint8)
        for off, (_n, a) in zip(self.offsets, self.tensors):
            if isinstance(a, RandI8):
                step = 1 << 24
                for c0 in range(0, a.size, step):
                    n = min(step, a.size - c0)
                    chunk = self.rng.integers(-127, 128, size=n, dtype=np.int8)
                    out[off + c0:off + c0 + n] = chunk.view(np.uint8)
            else:
                out[off:off + a.nbytes] = a.reshape(-1).view(np.uint8)

    def views(self, image: np.ndarray, base: int):
        """name -> int view of each tensor inside the written image."""
        res = {}
        for off, (n, a) in zip(self.offsets, self.tensors):
            dt = np.int8 if isinstance(a, RandI8) else a.dtype
            res[n] = image[base + off:base + off + a.nbytes].view(dt).reshape(a.shape)
        return res


def tensor_manifest(magic: bytes, elem_size: int, tensors) -> bytes:
    m = Manifest(magic, elem_size, tensors)
    out = np.zeros(m.size, dtype=np.uint8)
    m.write_into(out)
    return out.tobytes()


def kvc1(entries, value_words: int) -> bytes:
    """KVC1 keyed int64 tuples (docs/sslm_format.md:261-271)."""
    names = [n.encode() for n, _ in entries]
    name_blob = b"".join(names)
    out = bytearray(struct.pack("<4sIIIII", b"KVC1", 1, len(entries), value_words, len(name_blob), 0))
    off = 0
    for nb in names:
        out += struct.pack("<II", off, len(nb))
        off += len(nb)
    for _n, vals in entries:
        if len(vals) != value_words:
            raise ValueError("value_words mismatch")
        out += struct.pack(f"<{value_words}q", *[int(v) for v in vals])
    out += name_blob
    return bytes(out)


def cfg1(c: "ModelConfig") -> bytes:
    """CFG1 fixed 84-byte config (docs/sslm_format.md:301-321)."""
    return struct.pack("<4s16I2d", b"CFG1", 1, c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim,
                       c.inter, c.vocab, c.context_cap, 1 if c.tie_embeddings else 0, 0,
                       c.kv_block_size, 15, 0, 0, 0, c.rope_theta, 1e-6)


def sigmoid_lut() -> np.ndarray:
    """SIL1 nodes: round_half_even(sigmoid(-16 + i/32) * 2^15), i in [0, 1024]
    (docs/sslm_format.md:346-349), float64 as the converter computes it."""
    x = -16.0 + np.arange(1025, dtype=np.float64) * (32.0 / 1024.0)
    return np.rint((1.0 / (1.0 + np.exp(-x))) * 32768.0).astype(np.int32)


def sil1(table: np.ndarray) -> bytes:
    return struct.pack("<4sIII", b"SIL1", 1, 1025, 0) + np.asarray(table, dtype="<i4").tobytes()


def rope_tables(cap: int, head_dim: int, theta: float):
    """Q2.30 cos/sin [cap, head_dim/2] for interleaved pairs (2i, 2i+1), inv_freq theta^(-2i/d)."""
    pairs = head_dim // 2
    inv = theta ** (-(np.arange(pairs, dtype=np.float64) * 2.0) / head_dim)
    ang = np.arange(cap, dtype=np.float64)[:, None] * inv[None, :]
    one = float(1 << 30)
    return (np.rint(np.cos(ang) * one).astype(np.int64), np.rint(np.sin(ang) * one).astype(np.int64))


def scale_me(value: float):
    """Canonical carried scale (m, e): value = m * 2^e with m in [2^30, 2^31)."""
    if value <= 0:
        raise ValueError("scale must be positive")
    fr, ex = math.frexp(value)  # value = fr * 2^ex, fr in [0.5, 1)
    m = int(round(fr * (1 << 31)))
    e = ex - 31
    if m >= (1 << 31):
        m >>= 1
        e += 1
    return m, e


def reciprocal_round(m: int) -> int:
    """round_half_up(2^62 / m): KvLandingReciprocals word 2 for a landing mantissa m."""
    return ((1 << 63) + m) // (2 * m)


@dataclass
class ModelConfig:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    context_cap: int
    tie_embeddings: bool = True
    kv_block_size: int = 16
    rope_theta: float = 1_000_000.0
    with_bias: bool = False


CONFIGS = {
    # tiny shapes for CPU tests
    "tiny": ModelConfig(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=32, inter=256, vocab=512,
                        context_cap=64, tie_embeddings=False, with_bias=True),
    "small": ModelConfig(hidden=256, layers=3, heads=4, kv_heads=1, head_dim=64, inter=512, vocab=1024,
                         context_cap=160, tie_embeddings=True, with_bias=True),
    # wide enough that the decode GEMVs split K (hidden 1024, intermediate 2816)
    "medium": ModelConfig(hidden=1024, layers=2, heads=8, kv_heads=2, head_dim=128, inter=2816, vocab=4096,
                          context_cap=96, tie_embeddings=False, with_bias=True),
    # a context cap above one 512-token launch, for long prefill spans
    "long": ModelConfig(hidden=256, layers=2, heads=4, kv_heads=1, head_dim=64, inter=512, vocab=1024,
                        context_cap=1536, tie_embeddings=False, with_bias=True),
    # Qwen2.5-1.5B shape
    "qwen1.5b": ModelConfig(hidden=1536, layers=28, heads=12, kv_heads=2, head_dim=128, inter=8960,
                            vocab=151936, context_cap=1024, tie_embeddings=True),
    # Qwen2.5-7B shape
    "qwen7b": ModelConfig(hidden=3584, layers=28, heads=28, kv_heads=4, head_dim=128, inter=18944,
                          vocab=151936, context_cap=4608, tie_embeddings=False),
}


@dataclass
class SyntheticModel:
    config: ModelConfig
    weights: dict = field(default_factory=dict)    # name -> int8 ndarray
    folds: dict = field(default_factory=dict)      # name -> int32 [N,3]
    biases: dict = field(default_factory=dict)     # name -> int64 [N]
    consts: dict = field(default_factory=dict)     # name -> (m, e)
    landing: dict = field(default_factory=dict)    # "layer{l}.k_head{h}" -> (m, e, R)
    rope_cos: np.ndarray = None
    rope_sin: np.ndarray = None
    silu: np.ndarray = None

    image: np.ndarray = None
    rng: object = None
    # damped-greedy logit scale (m, e): written as a DampedGreedyConstants section with header
    # flag bit 1 (src/damped_greedy_phaseD.cpp: 12 raw bytes, int64 m then int32 e)
    damped: tuple = None
    # SCM1 schemas: [(name, {state: {token: next_state}}, accepting states)]
    schemas: list = None

    def to_bytes(self) -> bytes:
        return bytes(self.to_array())

    def to_array(self) -> np.ndarray:
        """The artifact file image as a uint8 array.  Built once; afterwards `weights` holds views
        into it (placeholders are drawn from the model's RNG in manifest order while writing)."""
        if self.image is None:
            self.image = self._write()
        return self.image

    def _write(self) -> np.ndarray:
        c = self.config
        wgt = Manifest(b"WGT1", 1, list(self.weights.items()))
        wgt.rng = self.rng
        wsc = Manifest(b"WSC1", 4, list(self.folds.items()))
        rop = Manifest(b"ROP1", 8, [("cos", self.rope_cos), ("sin", self.rope_sin)])
        comp = kvc1(list(self.consts.items()), 2)
        lscale = kvc1([(k, v[:2]) for k, v in self.landing.items()], 2)
        lrecip = kvc1(list(self.landing.items()), 3)
        sections = [
            (SEC_CONFIG, DT_RAW, cfg1(c), 8),
            (SEC_WEIGHTS, DT_I8, wgt, 64),
            (SEC_WEIGHT_SCALES, DT_I32, wsc, 64),
            (SEC_ROPE, DT_I64, rop, 64),
            (SEC_COMPOSITION, DT_RAW, comp, 8),
            (SEC_KV_LANDING_SCALES, DT_RAW, lscale, 8),
            (SEC_KV_LANDING_RECIPROCALS, DT_RAW, lrecip, 8),
            (SEC_SIGMOID_LUT, DT_I32, sil1(self.silu), 8),
        ]
        if self.biases:
            sections.append((SEC_BIASES, DT_I64, Manifest(b"BIA1", 8, list(self.biases.items())), 64))
        flags = 0
        if self.schemas:
            sections.append((SEC_SCHEMA_MASKS, DT_RAW, scm1(c.vocab, self.schemas), 8))
        if self.damped is not None:
            sections.append((SEC_DAMPED_GREEDY, DT_RAW, struct.pack("<qi", *self.damped), 8))
            flags |= 2
        img = write_container_array(sections, flags)
        base = int.from_bytes(img[HEADER_BYTES + SECTION_DESC_BYTES + 8:HEADER_BYTES + SECTION_DESC_BYTES + 16].tobytes(),
                              "little")  # offset of the Weights section (second in the table)
        self.weights.update(wgt.views(img, base))
        return img


def _fold_table(rng, n: int, shift_lo: int, shift_hi: int, identity_frac: float) -> np.ndarray:
    t = np.empty((n, 3), dtype=np.int32)
    t[:, 0] = (rng.random(n) < identity_frac).astype(np.int32)
    t[:, 1] = rng.integers(1 << 30, 1 << 31, size=n, dtype=np.int64).astype(np.int32)
    t[:, 2] = rng.integers(shift_lo, shift_hi + 1, size=n, dtype=np.int32)
    return t


def _codes(rng, shape):
    return RandI8(shape)


def build_synthetic(cfg: ModelConfig, seed: int = 1234, temperature: float = 1.0,
                    damped_logit_scale: float | None = None, schemas=None, edit=None) -> SyntheticModel:
    """Seeded synthetic integer model whose constants follow one real-scale model.

    Real value of a code = code * (m * 2^e).  Each projection's WSC1 fold F = acc * mult / 2^(31+s)
    carries unit x_scale * c_f with c_f = w_s * 2^31 / 2^30.5 (the shift and the per-channel mult
    spread act as per-channel weight-scale variation), so the projection site constant is c_f/127;
    norms use g_s / (2^16 * 127); residuals 1/127; the SiLU product 2^-15/127 (it already carries
    both incoming scales).  K/V land at a fixed code scale, and softmax_khead folds the k code
    scale with 1/sqrt(head_dim) so the derived i-exp q_ln2 sits near 5e4 score units.
    `damped_logit_scale` (the real value of one logit unit) adds the damped-greedy constants;
    `schemas` (see scm1) adds a SchemaMasks section.  `edit`, when given, is called with the
    model before its image is written (constants, folds and biases are still plain arrays)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    c = cfg
    m = SyntheticModel(config=c)
    if damped_logit_scale is not None:
        m.damped = scale_me(damped_logit_scale)
    m.schemas = schemas
    H, I, D, NH, NKV = c.hidden, c.inter, c.head_dim, c.heads, c.kv_heads
    KVH = NKV * D
    g_s = 1.0 / 127.0
    shift_lo, shift_hi = 0, 3
    mult_ref = 2.0 ** 30.5

    def c_f(k_in: int) -> float:
        w_s = 1.0 / (127.0 * math.sqrt(k_in))
        return w_s * 2.0 ** 31 / mult_ref

    m.weights["embed"] = _codes(rng, (c.vocab, H))
    m.consts["embed"] = scale_me(1.0 / 127.0 / 127.0)
    shapes = {"q_proj": (H, H), "k_proj": (KVH, H), "v_proj": (KVH, H), "o_proj": (H, H),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    k_code_scale = 1.5 / 127.0
    v_code_scale = 1.5 / 127.0
    for layer in range(c.layers):
        p = f"layer{layer}"
        for name in PROJECTIONS:
            m.weights[f"{p}.{name}"] = _codes(rng, shapes[name])
        m.weights[f"{p}.attn_norm.gain"] = _codes(rng, (H,))
        m.weights[f"{p}.mlp_norm.gain"] = _codes(rng, (H,))
        for name in PROJECTIONS:
            m.folds[f"{p}.{name}"] = _fold_table(rng, shapes[name][0], shift_lo, shift_hi, 0.03)
        m.folds[f"{p}.ctx_fold"] = _fold_table(rng, NH, 0, 2, 0.0)
        if c.with_bias:
            for name in ("q_proj", "k_proj", "v_proj"):
                b_real = rng.normal(0.0, 0.05, size=shapes[name][0])
                m.biases[f"{p}.{name}"] = np.rint(b_real * 2.0 ** 30 / c_f(H)).astype(np.int64)
        norm_site = scale_me(g_s / (2.0 ** 16 * 127.0))
        m.consts[f"{p}.attn_norm"] = norm_site
        m.consts[f"{p}.mlp_norm"] = norm_site
        for name in ("q_proj", "o_proj", "gate_proj", "up_proj"):
            m.consts[f"{p}.{name}"] = scale_me(c_f(H) / 127.0)
        m.consts[f"{p}.down_proj"] = scale_me(c_f(I) / 127.0)
        # ctx_wide = fold(sum p_q15 * v_code): unit v_code_scale * 2^31 / (mult * 2^15)
        m.consts[f"{p}.attn_ctx"] = scale_me(v_code_scale * 2.0 ** 31 / (mult_ref * 2.0 ** 15) / 127.0)
        m.consts[f"{p}.attn_residual"] = scale_me(1.0 / 127.0)
        m.consts[f"{p}.mlp_residual"] = scale_me(1.0 / 127.0)
        m.consts[f"{p}.mlp_act"] = scale_me(2.0 ** -15 / 127.0)
        for h in range(NKV):
            m.consts[f"{p}.softmax_khead{h}"] = scale_me(k_code_scale / math.sqrt(D) / temperature)
            for kind, code_scale in (("k", k_code_scale), ("v", v_code_scale)):
                # code = F * normed / landing  ->  landing = code_scale / c_f
                lm, le = scale_me(code_scale / c_f(H))
                m.landing[f"{p}.{kind}_head{h}"] = (lm, le, reciprocal_round(lm))
    m.weights["final_norm.gain"] = _codes(rng, (H,))
    m.consts["final_norm"] = scale_me(g_s / (2.0 ** 16 * 127.0))
    if not c.tie_embeddings:
        m.weights["lm_head"] = _codes(rng, (c.vocab, H))
    m.rope_cos, m.rope_sin = rope_tables(c.context_cap, D, c.rope_theta)
    m.silu = sigmoid_lut()
    m.rng = rng
    if edit is not None:
        edit(m)
    m.to_array()
    return m


def with_weight_rows(sm: SyntheticModel, name: str, rows: dict) -> bytes:
    """The image of `sm` with rows of weight tensor `name` replaced ({row index: int8 codes}) and
    the integrity hash recomputed; `sm` itself is left unchanged."""
    img = sm.to_array().copy()
    w = sm.weights[name]
    off = w.ctypes.data - sm.to_array().ctypes.data
    width = w.shape[1]
    for r, codes in rows.items():
        img[off + r * width:off + (r + 1) * width] = np.asarray(codes, dtype=np.int8).view(np.uint8)
    flags = int.from_bytes(img[16:20].tobytes(), "little")
    return with_flags(img.tobytes(), flags)


# ADP1 target-module bit order (reference include/superslm/model.h:433 kPeftAdaptableProjections)
PEFT_PROJECTIONS = ("q_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "k_proj", "v_proj")


def build_adapter(sm: SyntheticModel, rank: int = 16, targets=("q_proj", "v_proj"), seed: int = 77,
                  layers=None, name: str = "synthetic") -> bytes:
    """A seeded LoRA adapter artifact for `sm` (reference adapter_marshal.h PopulateAdapterFromView):
    Config and SigmoidLut copied from the base, Provenance = the 68-byte ADP1 record + name, Weights = "layer<N>.<proj>.lora_A" [rank, in] and
    ".lora_B" [out, rank] int8, DeltaFoldScales / UFoldScales = (identity, mult, exponent) rows
    for each adapted "layer<N>.<proj>".  The u folds bring A.x back into code range; the delta
    folds mix identity rows, attenuating exponents and amplifying (negative) exponents so every
    branch of the amplifying fold is exercised."""
    c = sm.config
    rng = np.random.default_rng(seed)
    base_hash = bytes(sm.to_array()[HASH_OFFSET:HASH_OFFSET + 32])
    kvh = c.kv_heads * c.head_dim
    out_ch = {"q_proj": c.hidden, "o_proj": c.hidden, "down_proj": c.hidden, "k_proj": kvh, "v_proj": kvh,
              "gate_proj": c.inter, "up_proj": c.inter}
    in_ch = {p: (c.inter if p == "down_proj" else c.hidden) for p in PEFT_PROJECTIONS}
    mask = 0
    for t in targets:
        mask |= 1 << PEFT_PROJECTIONS.index(t)
    weights, dfs, ufs = [], [], []
    for layer in (range(c.layers) if layers is None else layers):
        for proj in targets:
            key = f"layer{layer}.{proj}"
            k_in, n_out = in_ch[proj], out_ch[proj]
            a = rng.integers(-127, 128, size=(rank, k_in), dtype=np.int8)
            b = rng.integers(-127, 128, size=(n_out, rank), dtype=np.int8)
            # |A.x| ~ 127 * 73 * sqrt(K): exponent so u lands around +-40 (some rows saturate)
            ue = int(np.clip(np.round(np.log2(0.75 * 127 * 73 * np.sqrt(k_in) / 40.0)), 0, 31))
            u = np.empty((rank, 3), dtype=np.int32)
            u[:, 0] = 0
            u[:, 1] = rng.integers(1 << 30, 1 << 31, size=rank, dtype=np.int64).astype(np.int32)
            u[:, 2] = rng.integers(ue - 1, ue + 2, size=rank)
            u[rank // 2, 0] = 1  # one pass-through row (clamped to +-127 by the site)
            d = np.empty((n_out, 3), dtype=np.int32)
            d[:, 0] = (rng.random(n_out) < 0.1).astype(np.int32)
            d[:, 1] = rng.integers(1 << 30, 1 << 31, size=n_out, dtype=np.int64).astype(np.int32)
            d[:, 2] = rng.integers(-2, 9, size=n_out)
            weights += [(key + ".lora_A", a), (key + ".lora_B", b)]
            dfs.append((key, d))
            ufs.append((key, u))
    nm = name.encode()
    prov = struct.pack("<4siii32sdiii", b"ADP1", 1, rank, mask, base_hash, float(2 * rank), 0, 0, len(nm)) + nm
    sections = [  # the reference converter's six sections (tools/sslm_convert_adapter.py:1315-1320)
        (SEC_CONFIG, DT_RAW, cfg1(c), 8),
        (SEC_SIGMOID_LUT, DT_I32, sil1(sm.silu), 8),
        (SEC_PROVENANCE, DT_RAW, prov, 8),
        (SEC_WEIGHTS, DT_I8, Manifest(b"WGT1", 1, weights), 64),
        (SEC_DELTA_FOLD, DT_I32, Manifest(b"DFS1", 4, dfs), 64),
        (SEC_U_FOLD, DT_I32, Manifest(b"UFS1", 4, ufs), 64),
    ]
    return write_container(sections)
