"""Host orchestration of the DP clip kernels.

A ``GhostPlan`` turns one batch's captured layer inputs into problem tables
for the native kernels and runs the DP step as a fixed sequence of launches
on the current HIP stream:

    odp_project     U_i = G_i B_i^T, V = X [A_1 .. A_k]   (LoRA rank space)
    odp_seg_factor  per-example dA, dB and their squared-norm partials
    odp_sqnorm      squared norms of materialised per-example leaves
    odp_clip_factors  per-example norms -> clip / AUTO-S scales
    odp_scale_sum   clipped sum, cast and normalize_by, into one flat buffer

LoRA adapters that read the same activation tensor (q/k/v, gate/up) share
one pass over it: their ranks are laid side by side (up to 4 leaves and 64
columns per pass).  All metadata of a step is packed into one pinned host
buffer and uploaded with one asynchronous copy.
"""

from __future__ import annotations

import math
import struct
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from opaque_amd import _host

from opaque_amd import _native as N

_DTYPE_CODE = {torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16,
               torch.float64: N.DTYPE_F64}
_ALIGN = {torch.float32: 4, torch.bfloat16: 8}  # the LoRA and linear kernels' dtypes; 16-byte rows
MAX_RANK_PER_PASS = 64
MAX_LEAVES_PER_PASS = 4


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"opaque_amd kernels support float32, bfloat16, float16 and float64, got {dt}") from None


def _f64_bits(x: float) -> int:
    return struct.unpack("<q", struct.pack("<d", float(x)))[0]


def _rows(t: torch.Tensor) -> torch.Tensor:
    """2-D row view [rows, d] with unit column stride and a 16-byte aligned pitch."""
    t2 = t.reshape(-1, t.shape[-1])
    align = _ALIGN[t.dtype]
    if t2.stride(-1) != 1 or t2.stride(0) % align != 0 or t2.data_ptr() % 16 != 0:
        t2 = t2.contiguous()
    return t2


def supports_rows(t: torch.Tensor) -> bool:
    """Whether a [.., d] activation can go through the LoRA kernels."""
    return t.dtype in _ALIGN and t.shape[-1] % _ALIGN[t.dtype] == 0 and t.shape[-1] > 0


# ---------------------------------------------------------------------------
# Segments
# ---------------------------------------------------------------------------


@dataclass
class Segments:
    """Row ranges of examples (or (example, expert) pairs) in a row tensor."""

    starts: list[int]
    lengths: list[int]
    examples: list[int]
    n_ex: int
    n_rows: int

    def __post_init__(self) -> None:
        if not (len(self.starts) == len(self.lengths) == len(self.examples)):
            raise ValueError("segment arrays must have equal length")
        prev_end = 0
        for s, ln, e in zip(self.starts, self.lengths, self.examples):
            if ln < 0 or s < prev_end or s + ln > self.n_rows:
                raise ValueError(
                    f"segments must be sorted, non-overlapping and inside [0, {self.n_rows}); "
                    f"got start={s} len={ln} after end={prev_end}"
                )
            if not 0 <= e < self.n_ex:
                raise ValueError(f"segment example {e} outside [0, {self.n_ex})")
            prev_end = s + ln
        if self.n_rows >= 2**31 - 64:
            raise ValueError("row count exceeds the int32 segment range")

    @property
    def n_seg(self) -> int:
        return len(self.starts)

    @classmethod
    def padded(cls, n_ex: int, seq_len: int, lengths: list[int] | None = None) -> Segments:
        """Example i owns rows [i*seq_len, i*seq_len + lengths[i])."""
        lens = [seq_len] * n_ex if lengths is None else [int(x) for x in lengths]
        if len(lens) != n_ex or any(not 0 <= x <= seq_len for x in lens):
            raise ValueError("lengths must give one value in [0, seq_len] per example")
        return cls([i * seq_len for i in range(n_ex)], lens, list(range(n_ex)), n_ex, n_ex * seq_len)


def _pj_rows(dt: torch.dtype, v: "_SegView") -> int:
    """The rows odp_project's workgroups walk: the covered rows for bf16, all rows for f32."""
    return v.covered if dt == torch.bfloat16 else v.n_rows


@dataclass
class _SegView:
    """A segment list as laid out in the plan's device segment arrays."""

    segs: Segments
    first: int

    @property
    def n_seg(self) -> int:
        return self.segs.n_seg

    @property
    def n_rows(self) -> int:
        return self.segs.n_rows

    @property
    def valid(self) -> int:
        return int(sum(self.segs.lengths))

    @property
    def max_len(self) -> int:
        return max(self.segs.lengths, default=0)

    @property
    def covered(self) -> int:
        """Rows of the segments widened to whole 8-row groups (odp_project_covered_rows)."""
        return int(sum(((st + ln + 7) & ~7) - (st & ~7)
                       for st, ln in zip(self.segs.starts, self.segs.lengths) if ln > 0))


class _SegRegistry:
    """The plan's segments followed by every other segment list a site brings (MoE experts)."""

    def __init__(self, default: Segments) -> None:
        self.views: list[_SegView] = []
        self._by_id: dict[int, _SegView] = {}
        self.default = self.view(default)

    def view(self, segs: Segments | None) -> _SegView:
        if segs is None:
            return self.default
        v = self._by_id.get(id(segs))
        if v is None:
            if self.views and segs.n_ex != self.views[0].segs.n_ex:
                raise ValueError("all segment lists of a plan must count the same examples")
            if len(set(segs.examples)) != len(segs.examples):
                raise ValueError("each example may own at most one segment of a segment list")
            first = sum(w.n_seg for w in self.views)
            v = _SegView(segs, first)
            self.views.append(v)
            self._by_id[id(segs)] = v
        return v

    def arrays(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        st = np.asarray([x for v in self.views for x in v.segs.starts], dtype=np.int32)
        ln = np.asarray([x for v in self.views for x in v.segs.lengths], dtype=np.int32)
        ex = np.asarray([x for v in self.views for x in v.segs.examples], dtype=np.int32)
        return st.reshape(-1), ln.reshape(-1), ex.reshape(-1)


# ---------------------------------------------------------------------------
# Inputs and outputs of a plan
# ---------------------------------------------------------------------------


@dataclass
class LoraSite:
    """One LoRA application y = x W^T + s (x A) B over the batch rows.

    ``A`` is [d_in, r] and ``B`` is [r, d_out] (kernel convention).  The
    gradient leaves are indices into the plan's leaf list (None when the
    factor is frozen); ``a_transposed`` / ``b_transposed`` say that the leaf
    is stored as [r, d_in] / [d_out, r] (PEFT's lora_A.weight/lora_B.weight).
    """

    x: torch.Tensor
    g: torch.Tensor
    A: torch.Tensor
    B: torch.Tensor
    scaling: float
    a_leaf: int | None
    b_leaf: int | None
    a_transposed: bool = False
    b_transposed: bool = False
    segments: Segments | None = None  # rows of x / g; None: the plan's segments
    # The seam's own rank-space products, when it kept them: v = x A (its
    # forward) and u = g B^T (its input-gradient backward), [rows, r] in
    # x's dtype.  With both, for every site of an activation, the plan reads
    # them instead of projecting X and G again.
    v: torch.Tensor | None = None
    u: torch.Tensor | None = None


def _seam_rows(t: torch.Tensor) -> torch.Tensor:
    """2-D row view [rows, r] of a seam product with unit column stride."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def uses_seam_products(chunk: list[LoraSite]) -> bool:
    """Whether the sites of one activation all bring both seam products in
    the activation's dtype, one row per activation row."""
    x = chunk[0].x
    dt, n_rows = x.dtype, x.numel() // max(x.shape[-1], 1)
    for s in chunk:
        r = s.A.shape[1]
        for t in (s.v, s.u):
            if t is None or t.dtype != dt or t.device != s.x.device or t.dim() < 1 or t.shape[-1] != r \
                    or t.numel() != n_rows * r:
                return False
    return True


# Addresses per LoRA site that plan_key writes to ``lora_ptrs``: x, g, A, B, v, u.
LORA_PTRS = 6


@dataclass
class LinearSite:
    """A full-weight linear y = x W^T over the batch rows (bf16).

    ``w_leaf`` indexes the plan's leaf list; the leaf is W's gradient,
    shaped [d_out, d_in], or with ``index`` one slice of a stacked
    [E, d_out, d_in] leaf (each slice produced by one site).  ``form`` picks the per-example norm algorithm
    (``N.FORM_OUTER`` / ``N.FORM_GRAM``; ``N.FORM_GRAM256`` forces the
    256-row-block Gram kernel); None chooses the one with fewer MFMA flops
    for the longest segment.
    """

    x: torch.Tensor
    g: torch.Tensor
    w_leaf: int
    form: int | None = None
    segments: Segments | None = None  # rows of x / g; None: the plan's segments
    index: int | None = None  # slice of a stacked [E, d_out, d_in] leaf (an MoE expert); None: the whole leaf


# Time per flop of the Gram-form norm kernel relative to the outer form,
# measured on MI355X (C4 shapes: 1264 vs 746 TFLOP/s).
GRAM_FLOP_COST = 1.6

# A site in the Gram form whose longest segment spans at least
# GRAM256_MIN_LEN rows takes the 256-row-block kernel (N.FORM_GRAM256: fewer
# loads per flop) while its scratch, GRAM256_ITEM_BYTES per segment and block
# pair, fits within GRAM256_SCRATCH_BYTES and a quarter of the free device
# memory at plan build; the others take the 128-row-block kernel.
GRAM256_MIN_LEN = 512
GRAM256_SCRATCH_BYTES = 32 << 30
GRAM256_ITEM_BYTES = 256 * 256 * 4
# Its time per flop relative to the outer form, measured on MI355X (C4
# gate/up/down at 4096 tokens: 1090 vs 1233-1262 TFLOP/s).
GRAM256_FLOP_COST = 1.15


def split_budget(avail: int | None, stored: int, prescale_bytes: int) -> tuple[int, int]:
    """(Gram scratch bytes, prescaled-activation bytes) a plan may use, from
    the device memory available when it is built (``avail``; None off the
    GPU: no device limit) once ``stored`` bytes of per-example gradients are
    placed.  The 256-row Gram kernels' scratch gets up to a quarter of the
    rest (and at most GRAM256_SCRATCH_BYTES), the prescaled activations up
    to half of what then remains (and at most ``prescale_bytes``), so the
    three together never exceed ``avail``."""
    if avail is None:
        return GRAM256_SCRATCH_BYTES, prescale_bytes
    rest = max(0, avail - stored)
    scr = min(GRAM256_SCRATCH_BYTES, rest // 4)
    return scr, min(prescale_bytes, (rest - scr) // 2)


def choose_form(max_len: int, d_in: int, d_out: int) -> int:
    """The faster form: GRAM costs L^2 (d_in + d_out) flops per example (upper
    triangle) at GRAM_FLOP_COST (GRAM256_FLOP_COST from GRAM256_MIN_LEN rows)
    times the outer kernel's time per flop, OUTER 2 L d_in d_out."""
    cost = GRAM256_FLOP_COST if max_len >= GRAM256_MIN_LEN else GRAM_FLOP_COST
    return N.FORM_GRAM if cost * max_len * (d_in + d_out) < 2 * d_in * d_out else N.FORM_OUTER


@dataclass
class MaterializedLeaf:
    """A leaf whose per-example gradients are already materialised: [n_seg, *shape]."""

    per_example: torch.Tensor
    leaf: int
    segments: Segments | None = None  # one row of per_example per segment; None: the plan's


@dataclass
class LeafOut:
    shape: tuple[int, ...]
    out_dtype: torch.dtype
    group: int = 0
    cls: int = 0


@dataclass
class ClipSpec:
    mode: int  # N.CLIP_FIXED or N.CLIP_AUTOS
    thresholds: list[float]  # per group
    effective: float
    gamma: float = 0.01
    normalize_by: float = 1.0
    guards: list[tuple[float, float, torch.dtype]] = field(default_factory=list)  # per cls


@dataclass
class GhostResult:
    leaves: list[torch.Tensor]
    norms: torch.Tensor  # [n_ex] f32
    group_norms: torch.Tensor  # [G, n_ex] f32
    clipped: torch.Tensor  # [G, n_ex] uint8
    clipped_total: torch.Tensor  # [n_ex] uint8
    scales: torch.Tensor  # [n_cls, G, n_ex] f64 (each value as its class dtype holds it)
    second_moment: list[torch.Tensor] | None
    flat: dict[torch.dtype, torch.Tensor]


class _Pack:
    """Collects host arrays and uploads them with one pinned async copy."""

    def __init__(self) -> None:
        self._chunks: list[np.ndarray] = []
        self._offsets: list[int] = []
        self._size = 0

    def add(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        off = (self._size + 255) // 256 * 256
        self._chunks.append(arr)
        self._offsets.append(off)
        self._size = off + arr.nbytes
        return len(self._chunks) - 1

    def array(self, i: int) -> np.ndarray:
        return self._chunks[i]

    def _pinned(self) -> torch.Tensor:
        host = torch.empty(max(self._size, 1), dtype=torch.uint8, pin_memory=True)
        hn = host.numpy()
        for arr, off in zip(self._chunks, self._offsets):
            hn[off : off + arr.nbytes] = arr.view(np.uint8).reshape(-1)
        return host

    def refresh(self) -> None:
        """Copies the (patched) host arrays into the same device buffer.  The
        copy is ordered on the current stream after earlier launches that read
        the buffer; torch's pinned-memory allocator keeps the source alive
        until the copy is done."""
        self._dev.copy_(self._pinned(), non_blocking=True)

    def upload(self, device: torch.device) -> list[torch.Tensor]:
        dev = self._pinned().to(device, non_blocking=True)
        self._dev = dev
        views = []
        for arr, off in zip(self._chunks, self._offsets):
            tdt = {
                np.dtype(np.int64): torch.int64,
                np.dtype(np.int32): torch.int32,
                np.dtype(np.float64): torch.float64,
            }[arr.dtype]
            views.append(dev[off : off + arr.nbytes].view(tdt))
        return views


class _Table:
    def __init__(self, fields: int) -> None:
        self.fields = fields
        self.rows: list[list[int]] = []
        self.blocks: list[int] = []
        self.nbytes = 0  # algorithmic HBM bytes of the launch (one read/write of each operand)
        self.nflops = 0  # algorithmic flops of the launch
        # The part of nbytes that the step's contract counts: reads of the
        # activations and output gradients (and of materialised per-example
        # gradients), and the clipped sums written; not the plan's own
        # intermediates (rank-space planes, stored per-example gradients).
        self.io_bytes = 0

    def add(self, row: dict[int, int], blocks: int, nbytes: int = 0, nflops: int = 0, io: int = 0) -> None:
        if blocks <= 0:
            return
        self.nbytes += int(nbytes)
        self.nflops += int(nflops)
        self.io_bytes += int(io)
        r = [0] * self.fields
        for k, v in row.items():
            r[k] = int(v)
        self.rows.append(r)
        self.blocks.append(int(blocks))

    def arrays(self) -> tuple[np.ndarray, np.ndarray, int]:
        probs = np.asarray(self.rows, dtype=np.int64).reshape(-1, self.fields)
        ws = np.zeros(len(self.blocks) + 1, dtype=np.int64)
        np.cumsum(self.blocks, out=ws[1:])
        total = int(ws[-1])
        if total >= 2**31 - 1:
            raise ValueError("launch exceeds the int32 workgroup range; split the batch")
        return probs, ws.astype(np.int32), total


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream



def _layout(ext: dict[tuple, torch.Tensor]) -> list[tuple]:
    """Shapes, strides, dtypes and storage sharing of a plan's input tensors:
    a new call's inputs may replace them only if this matches."""
    storages: dict[int, int] = {}
    out = []
    for k, t in ext.items():
        base = t.untyped_storage().data_ptr()
        out.append((k, tuple(t.shape), tuple(t.stride()), t.dtype, storages.setdefault(base, len(storages)),
                    t.data_ptr() - base))
    return out


def _seg_key(segs: Segments | None) -> tuple | None:
    if segs is None:
        return None
    return (tuple(segs.starts), tuple(segs.lengths), tuple(segs.examples), segs.n_ex, segs.n_rows)


def _tensor_key(t: torch.Tensor) -> tuple:
    return (t.shape, t.stride(), t.dtype, t.get_device(), t.data_ptr() & 15)


def leaves_key(leaves: list[LeafOut]) -> tuple:
    """The part of plan_key that the output leaves fix (callers that reuse
    one leaf list may compute it once and pass it to plan_key)."""
    return tuple((tuple(lf.shape), lf.out_dtype, lf.group, lf.cls) for lf in leaves)


# GhostPlan's keyword options and their defaults (part of a plan's key).
_PLAN_OPTIONS = {"second_moment": False, "fuse_g_side": True, "stream_factors": True, "prescale_bytes": 8 << 30,
                 "linear_pe_bytes": None, "square_f64": False, "sum_f64": False, "raw_values": False}


def plan_key(*, segments: Segments, leaves: list[LeafOut], clip: ClipSpec, lora_sites=(), materialized=(),
             linear_sites=(), device=None, leaves_key_: tuple | None = None, lora_ptrs: torch.Tensor | None = None,
             **options) -> tuple:
    """What fixes a GhostPlan's tables: a plan built from inputs with this key
    can be rebound (GhostPlan.rebind) to other inputs with the same key.
    Threshold values, gamma and normalize_by are not part of it.

    With the host helper built, the LoRA sites' part is its byte signature
    (the same fields), and ``lora_ptrs`` (an int64 CPU tensor of at least
    LORA_PTRS entries per LoRA site) receives the addresses of each site's
    x, g, A, B, v and u (0 for a missing product) for rebind()."""
    host = _host.load()
    lora_sig = None
    if host is not None:
        buf = lora_ptrs if lora_ptrs is not None else torch.empty(LORA_PTRS * len(lora_sites), dtype=torch.int64)
        lora_sig = host.lora_signature(list(lora_sites), buf)
    firsts: dict[int, int] = {}
    xkeys: list[tuple] = []

    def shared(t: torch.Tensor):  # index of the first site input at this address
        p = t.data_ptr()
        i = firsts.get(p)
        if i is None:
            i = firsts[p] = len(xkeys)
            xkeys.append(_tensor_key(t))
            return i
        k = _tensor_key(t)
        return i if k == xkeys[i] else (i, k)  # another view at the same address

    # odp_pack_factors reads A with the strides and dtype in its table; B is
    # copied into the activation's dtype unless it can be read in place.
    if lora_sig is not None:
        lora = ("host", lora_sig)
    else:
        lora = tuple((shared(s.x), _tensor_key(s.g), _tensor_key(s.A), s.B.shape, s.B.get_device(),
                      s.B.dtype, s.B.is_contiguous(), float(s.scaling), s.a_leaf, s.b_leaf, s.a_transposed,
                      s.b_transposed, None if s.segments is None else _seg_key(s.segments),
                      None if s.v is None else _tensor_key(s.v), None if s.u is None else _tensor_key(s.u))
                     for s in lora_sites)
    mats = tuple((_tensor_key(m.per_example), m.leaf, _seg_key(m.segments)) for m in materialized)
    lins = tuple((shared(ls.x), _tensor_key(ls.g), ls.w_leaf, ls.form, ls.index,
                  _seg_key(ls.segments)) for ls in linear_sites)
    outs = leaves_key(leaves) if leaves_key_ is None else leaves_key_
    clip_s = (clip.mode, len(clip.thresholds), tuple(g[2] for g in clip.guards))
    unknown = set(options) - set(_PLAN_OPTIONS)
    if unknown:
        raise TypeError(f"unknown GhostPlan options {sorted(unknown)}")
    opts = tuple((k, options.get(k, v)) for k, v in _PLAN_OPTIONS.items())
    dev = torch.device(device) if device is not None else None
    if dev is not None and dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return (str(dev), _seg_key(segments), outs, clip_s, tuple(xkeys), lora, mats, lins, opts)


# ---------------------------------------------------------------------------
# The plan
# ---------------------------------------------------------------------------


# Stages launched after the clip factors, in table order.
_AFTER_CLIP = ("scale_sum", "lin_prescale", "lin_sum", "lin_moments")


class GhostPlan:
    """Buffers and problem tables of one DP clip step.  Build, then ``run()``.

    A plan may be run repeatedly (the bench does) as long as the tensors it
    was built from stay alive and unchanged in shape.

    ``fuse_g_side``: LoRA sites take the single-pass kernels where they can
    (results are bit-identical either way).  ``stream_factors``: bf16
    factor problems whose leaves each take a 16-row block of the rank plane
    (rank <= 16, at most three blocks) take odp_seg_factor_stream instead of
    odp_seg_factor (bit-identical).  ``linear_pe_bytes``: HBM for
    the stored per-example gradients of full-weight sites (bf16); None uses
    half of the free device memory, 0 stores none.  ``prescale_bytes``: at
    most this much of prescaled activations per clipped-sum chunk.
    ``square_f64``: materialised leaves are squared in float64 (the
    reference's accumulation dtype when a leaf is float64 or
    compute_dtype=float64); ``sum_f64``: the clipped sums of stored
    gradients accumulate in float64 (compute_dtype=float64).
    ``raw_values``: the materialised leaves hold values a caller's scale
    function already scaled: they are summed as they are (scale 1, non-finite
    entries kept) and their norms taken without nan_to_num.
    ``second_moment``: the plan also sums the squared clipped per-example
    gradients; full-weight sites whose gradients are not stored then take
    the moments kernel instead of the clipped-sum GEMM (both sums in float32).
    """

    def __init__(
        self,
        *,
        segments: Segments,
        leaves: list[LeafOut],
        clip: ClipSpec,
        lora_sites: list[LoraSite] = (),
        materialized: list[MaterializedLeaf] = (),
        linear_sites: list[LinearSite] = (),
        device: torch.device | str = "cuda",
        second_moment: bool = False,
        fuse_g_side: bool = True,
        stream_factors: bool = True,
        prescale_bytes: int = 8 << 30,
        linear_pe_bytes: int | None = None,
        square_f64: bool = False,
        sum_f64: bool = False,
        raw_values: bool = False,
    ) -> None:
        t_build = time.perf_counter()
        N.load()
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.segments = segments
        self.leaves = leaves
        self.clip = clip
        self.second_moment = second_moment
        self.fuse_g_side = fuse_g_side
        self.stream_factors = bool(stream_factors)
        self.prescale_bytes = int(prescale_bytes)
        self.linear_pe_bytes = linear_pe_bytes
        self.square_f64 = bool(square_f64)
        self.sum_f64 = bool(sum_f64)
        self.raw_values = bool(raw_values)
        self.n_groups = len(clip.thresholds)
        self.n_cls = max(1, len(clip.guards))
        if self.n_groups < 1:
            raise ValueError("at least one clip group is required")
        if self.n_cls > 8:
            raise ValueError("at most 8 storage dtype classes")
        for lf in leaves:
            if not 0 <= lf.group < self.n_groups or not 0 <= lf.cls < self.n_cls:
                raise ValueError("leaf group/class out of range")
        self._keep: list[torch.Tensor] = []
        # The structure this plan was built for: rebind(key=...) with an equal
        # key skips re-deriving the input layout.
        self.key = plan_key(segments=segments, leaves=leaves, clip=clip, lora_sites=lora_sites,
                            materialized=materialized, linear_sites=linear_sites, device=dev,
                            second_moment=second_moment, fuse_g_side=fuse_g_side, stream_factors=stream_factors,
                            prescale_bytes=prescale_bytes,
                            linear_pe_bytes=linear_pe_bytes, square_f64=square_f64, sum_f64=sum_f64,
                            raw_values=raw_values)
        self._build(list(lora_sites), list(materialized), list(linear_sites))
        self.build_ms = (time.perf_counter() - t_build) * 1e3  # host time of the construction

    # -- construction --------------------------------------------------------
    def _build(self, sites: list[LoraSite], mats: list[MaterializedLeaf], lins: list[LinearSite]) -> None:
        seg = self.segments
        dev = self.device
        reg = _SegRegistry(seg)
        self._segreg = reg
        for ls in lins:
            if ls.x.device != dev or ls.g.device != dev:
                raise ValueError("linear site tensors must be on the plan device")
            if ls.x.dtype != torch.bfloat16 or ls.g.dtype != torch.bfloat16:
                raise TypeError("full-weight linear sites run in bfloat16")
            n_rows = reg.view(ls.segments).n_rows
            if ls.x.reshape(-1, ls.x.shape[-1]).shape[0] != n_rows or \
                    ls.g.reshape(-1, ls.g.shape[-1]).shape[0] != n_rows:
                raise ValueError("linear site row count does not match the segments")
            if not (supports_rows(ls.x) and supports_rows(ls.g)):
                raise ValueError("linear site feature sizes must be multiples of 8")
            # The kernels address one segment's rows through 32-bit buffer ranges.
            ld = max(_rows(ls.x).stride(0), _rows(ls.g).stride(0))
            if reg.view(ls.segments).max_len * ld * 2 >= 2**31:
                raise ValueError("a linear site's longest segment spans 2 GiB or more of x or g")
            shape = tuple(self.leaves[ls.w_leaf].shape)
            want = (ls.g.shape[-1], ls.x.shape[-1])
            if ls.index is None and shape != want:
                raise ValueError("a linear site's leaf must be shaped [d_out, d_in]")
            if ls.index is not None and (len(shape) != 3 or shape[1:] != want or not 0 <= ls.index < shape[0]):
                raise ValueError("a stacked linear site's leaf must be shaped [E, d_out, d_in] with index < E")
        # Group sites by activation tensor, then chunk by rank/leaf budget.
        for s in sites:
            if s.x.device != dev or s.g.device != dev or s.A.device != dev or s.B.device != dev:
                raise ValueError("LoRA site tensors must be on the plan device")
            if s.x.dtype != s.g.dtype:
                raise TypeError("x and g of a LoRA site must share a dtype")
            n_rows = reg.view(s.segments).n_rows
            if s.x.reshape(-1, s.x.shape[-1]).shape[0] != n_rows or s.g.reshape(-1, s.g.shape[-1]).shape[0] != n_rows:
                raise ValueError("LoRA site row count does not match the segments")
            if not (supports_rows(s.x) and supports_rows(s.g)):
                raise ValueError("LoRA site feature sizes must be multiples of 8 (bf16) / 4 (f32)")
        groups: dict[tuple, list[LoraSite]] = {}
        for s in sites:
            if s.a_leaf is None and s.b_leaf is None:
                continue
            k = (s.x.data_ptr(), tuple(s.x.shape), tuple(s.x.stride()), s.x.dtype, reg.view(s.segments).first)
            groups.setdefault(k, []).append(s)
        chunks: list[list[LoraSite]] = []
        for members in groups.values():
            cur: list[LoraSite] = []
            rtot = 0
            for s in members:
                r = s.A.shape[1]
                if r > MAX_RANK_PER_PASS:
                    raise ValueError(f"LoRA rank {r} exceeds {MAX_RANK_PER_PASS}")
                if cur and (len(cur) == MAX_LEAVES_PER_PASS or rtot + r > MAX_RANK_PER_PASS):
                    chunks.append(cur)
                    cur, rtot = [], 0
                cur.append(s)
                rtot += r
            if cur:
                chunks.append(cur)
        # The tables point into tensors that come from the caller's inputs
        # (row views of x and g, weight copies, materialised leaves), each
        # made once under a key that rebind() reproduces from the next
        # call's inputs.
        site_index = {id(s): k for k, s in enumerate(sites)}
        self._chunk_sites = [[site_index[id(s)] for s in ch] for ch in chunks]
        # Chunks whose sites bring the seam's V and U skip the projections.
        self._chunk_products = [uses_seam_products(ch) for ch in chunks]
        self._lwx_groups = self._factor_groups(chunks, self._chunk_products)
        self._ext_keys = self._external_keys(chunks, len(mats), len(lins))
        ext = dict(zip(self._ext_keys, self._external_list(chunks, mats, lins)))
        self._ext = ext
        self._layout_in = _layout(ext)
        # Tensors that are their input itself or a view at the same address
        # (no copy was made): with an equal plan key the next call's input
        # stands in for the view (rebind's fast path).
        src = self._ext_sources(chunks, mats, lins)
        self._direct = [k in src and ext[k].data_ptr() == src[k].data_ptr() for k in self._ext_keys]
        self._fast = self._fast_map(chunks, ext, len(sites))
        # A^T of every chunk's sites, [sum of ranks][d_in] in the activation
        # dtype: plan scratch that odp_pack_factors fills from the caller's A
        # at the start of every run (one buffer per (dtype, d_in) group).
        lib = N.load()
        self._lwx_bufs = []
        wx_of: dict[int, torch.Tensor] = {}
        pft = _Table(N.PF_FIELDS)
        for cis in self._lwx_groups:
            dt = chunks[cis[0]][0].x.dtype
            d_in = chunks[cis[0]][0].A.shape[0]
            rows = sum(s.A.shape[1] for ci in cis for s in chunks[ci])
            buf = torch.empty((rows, d_in), dtype=dt, device=dev)
            self._lwx_bufs.append(buf)
            r0 = 0
            for ci in cis:
                rtot = sum(s.A.shape[1] for s in chunks[ci])
                wx_of[ci] = buf[r0 : r0 + rtot]
                c0 = 0
                for j, s in enumerate(chunks[ci]):
                    A = ext[("la", ci, j)]
                    r = A.shape[1]
                    pft.add({N.PF_SRC: A.data_ptr(), N.PF_LD0: A.stride(0), N.PF_LD1: A.stride(1),
                             N.PF_DTYPES: dtype_code(A.dtype) | (dtype_code(dt) << 8), N.PF_DIN: d_in, N.PF_R: r,
                             N.PF_DST: buf[r0 + c0 : r0 + c0 + r].data_ptr()},
                            lib.odp_pack_factors_blocks(d_in), d_in * r * (A.element_size() + buf.element_size()))
                    c0 += r
                r0 += rtot
        lin_x = [ext[("linx", i)] for i in range(len(lins))]
        lin_g = [ext[("ling", i)] for i in range(len(lins))]

        # Slot allocation: leaf -> number of partial slots, assigned in group order.
        leaf_slots: dict[int, int] = {}
        pe_elems: dict[int, int] = {}
        leaf_rank_m: dict[int, tuple[int, int]] = {}
        lib = N.load()
        leaf_view: dict[int, _SegView] = {}
        pe_dt: dict[int, torch.dtype] = {}
        for ch in chunks:
            dcode = dtype_code(ch[0].x.dtype)
            rtot = sum(s.A.shape[1] for s in ch)
            fused = len({s.scaling for s in ch if s.a_leaf is not None}) <= 1
            n_seg = reg.view(ch[0].segments).n_seg
            for s in ch:
                for lf in (s.a_leaf, s.b_leaf):
                    if lf is not None:
                        leaf_view[lf] = reg.view(s.segments)
                        # Stored per-example factor gradients in the parameter dtype.
                        pe_dt[lf] = ch[0].x.dtype
                d_in, r = s.A.shape
                d_out = s.B.shape[1]
                if s.a_leaf is not None:
                    # dA leaves of one activation share a pass of width rtot.
                    leaf_slots[s.a_leaf] = N.FT_WAVE_SLOTS * int(
                        lib.odp_seg_factor_tiles(dcode, d_in, rtot if fused else r))
                    leaf_rank_m[s.a_leaf] = (r, d_in)
                    pe_elems[s.a_leaf] = n_seg * r * d_in
                if s.b_leaf is not None:
                    leaf_slots[s.b_leaf] = N.FT_WAVE_SLOTS * int(lib.odp_seg_factor_tiles(dcode, d_out, r))
                    leaf_rank_m[s.b_leaf] = (r, d_out)
                    pe_elems[s.b_leaf] = n_seg * r * d_out
        for m in mats:
            n = int(math.prod(m.per_example.shape[1:]))
            leaf_view[m.leaf] = reg.view(m.segments)
            if m.per_example.shape[0] != leaf_view[m.leaf].n_seg:
                raise ValueError("materialised leaves need one row per segment")
            leaf_slots[m.leaf] = int(N.load().odp_sqnorm_blocks(n))
        # Linear sites: per site its norm form, segment view and first partial
        # slot within its leaf (the slices of a stacked leaf follow each other).
        # Sites whose per-example gradients fit in linear_pe_bytes keep them:
        # the outer form stores them (bf16) as it computes the norms, and
        # the clipped sum becomes a pass over storage.  That beats the Gram
        # form, which would still need the clipped-sum GEMM, whatever the
        # sequence length.  The other sites take the faster norm form and
        # the GEMM.
        # One reading of the device memory available to the plan (free plus
        # what torch's allocator holds unused, e.g. an earlier plan's
        # buffers, so repeated calls see the same budgets) is shared by the
        # stored gradients, the Gram scratch and the prescaled activations.
        avail = 0
        if dev.type == "cuda" and lins:
            cached = torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev)
            avail = torch.cuda.mem_get_info(dev)[0] + cached
        budget = self.linear_pe_bytes if self.linear_pe_bytes is not None else avail // 2
        lin_pe: dict[int, int] = {}  # site -> element offset in self.lin_pe
        pe_total = 0
        for i, ls in enumerate(lins):
            v = reg.view(ls.segments)
            n = v.n_seg * ls.x.shape[-1] * ls.g.shape[-1]
            if ls.form in (None, N.FORM_OUTER) and (pe_total + n) * 2 <= budget:
                lin_pe[i] = pe_total
                pe_total += (n + 127) // 128 * 128
        scr_budget, self._prescale_budget = split_budget(avail if dev.type == "cuda" else None, 2 * pe_total,
                                                         self.prescale_bytes)
        lin_scr: dict[int, int] = {}  # site -> byte offset in self.gram_scr (GRAM256 sites)
        scr_total = 0
        lin_form: list[int] = []
        lin_view: list[_SegView] = []
        lin_off: list[int] = []
        lin_goff: dict[int, int] = {}  # Gram site -> first slot of its guarded outer-form partials
        others = set(leaf_slots)
        slices: dict[int, set[int]] = {}
        for i, ls in enumerate(lins):
            d_in, d_out = ls.x.shape[-1], ls.g.shape[-1]
            v = reg.view(ls.segments)
            if i in lin_pe:
                form = N.FORM_OUTER
            else:
                form = ls.form if ls.form is not None else choose_form(v.max_len, d_in, d_out)
            if (form == N.FORM_GRAM and v.max_len >= GRAM256_MIN_LEN) or form == N.FORM_GRAM256:
                need = v.n_seg * int(lib.odp_linear_tiles(N.FORM_GRAM256, d_in, d_out, v.max_len)) \
                    * GRAM256_ITEM_BYTES
                if form == N.FORM_GRAM256 or scr_total + need <= scr_budget:
                    form = N.FORM_GRAM256
                    lin_scr[i] = scr_total
                    scr_total += need
            tiles = int(lib.odp_linear_tiles(form, d_in, d_out, v.max_len))
            lin_form.append(form)
            lin_view.append(v)
            taken = slices.setdefault(ls.w_leaf, set())
            key = -1 if ls.index is None else ls.index
            if ls.w_leaf in others or key in taken or (taken and (key == -1) != (-1 in taken)):
                raise ValueError(f"leaf {ls.w_leaf} (slice {ls.index}) has more than one producer")
            taken.add(key)
            lin_off.append(leaf_slots.get(ls.w_leaf, 0))
            leaf_slots[ls.w_leaf] = leaf_slots.get(ls.w_leaf, 0) + tiles
            if form in (N.FORM_GRAM, N.FORM_GRAM256):
                # Outer-form slots for the segments whose Gram products could
                # overflow float32 (odp_linear_sqnorm, ODP_FORM_OUTER_GUARDED).
                lin_goff[i] = leaf_slots[ls.w_leaf]
                leaf_slots[ls.w_leaf] += int(lib.odp_linear_tiles(N.FORM_OUTER_GUARDED, d_in, d_out, v.max_len))
        for k, taken in slices.items():
            if -1 not in taken and taken != set(range(self.leaves[k].shape[0])):
                raise ValueError(f"stacked leaf {k} needs a linear site for every slice")
        if set(leaf_slots) != set(range(len(self.leaves))):
            missing = sorted(set(range(len(self.leaves))) - set(leaf_slots))
            raise ValueError(f"every output leaf needs exactly one producer; missing {missing}")
        order = sorted(leaf_slots, key=lambda i: (self.leaves[i].group, i))
        slot_base: dict[int, int] = {}
        gstart = np.zeros(self.n_groups + 1, dtype=np.int64)
        pos = 0
        for i in order:
            slot_base[i] = pos
            pos += leaf_slots[i]
            gstart[self.leaves[i].group + 1] = pos
        for g in range(1, self.n_groups + 1):  # empty groups
            gstart[g] = max(gstart[g], gstart[g - 1])
        self.n_slots = max(pos, 1)

        # Device buffers.  Per-example factor gradients: one buffer per dtype.
        pe_off: dict[int, int] = {}
        pe_size: dict[torch.dtype, int] = {}
        for i in sorted(pe_elems):
            pe_off[i] = pe_size.get(pe_dt[i], 0)
            pe_size[pe_dt[i]] = pe_off[i] + (pe_elems[i] + 63) // 64 * 64
        self.pe = {dt: torch.empty(n, dtype=dt, device=dev) for dt, n in pe_size.items()}
        self._pe_slices = [(pe_dt[i], pe_off[i], pe_elems[i]) for i in sorted(pe_elems)]

        def pe_addr(i: int) -> int:
            buf = self.pe[pe_dt[i]]
            return buf.data_ptr() + pe_off[i] * buf.element_size()

        def pe_bits(i: int) -> int:  # the leaf descriptor's dtype bit
            return (1 << 32) if pe_dt[i] == torch.bfloat16 else 0

        self._pe_addr, self._pe_bits = pe_addr, pe_bits
        # fp64 partials [n_ex][n_slots], then one word that kernels set when a
        # per-example weight gradient held a non-finite entry; zeroed together.
        self._part_buf = torch.zeros(seg.n_ex * self.n_slots + 1, dtype=torch.float64, device=dev)
        self.part = self._part_buf[: seg.n_ex * self.n_slots].view(seg.n_ex, self.n_slots)
        self._nf_flag_addr = self._part_buf.data_ptr() + seg.n_ex * self.n_slots * 8

        ext.update(self._alloc_outputs())

        # Q planes (U and V) for every chunk, carved from one allocation per dtype.
        q_need: dict[torch.dtype, int] = {}
        chunk_layout = []
        for ch in chunks:
            dt = ch[0].x.dtype
            rtot = sum(s.A.shape[1] for s in ch)
            rows_alloc = (rtot + 15) // 16 * 16 + 16
            planes = 1  # one plane in the activation dtype (bf16: the reference's rounding of X A, G B^T)
            ldq = (reg.view(ch[0].segments).n_rows + 32 + 7) // 8 * 8
            per = planes * rows_alloc * ldq
            base = q_need.get(dt, 0)
            chunk_layout.append((dt, rtot, rows_alloc, planes, base, base + per, ldq))
            q_need[dt] = base + 2 * per
        self.qbuf = {dt: torch.empty(max(n, 1), dtype=dt, device=dev) for dt, n in q_need.items()}
        # Where each LoRA site's columns of the V and U planes lie (rank_planes).
        self._planes_of: dict[int, tuple] = {}
        for ci, (ch, (dt, _, _, _, vbase, ubase, ldq)) in enumerate(zip(chunks, chunk_layout)):
            c0 = 0
            for j, s in enumerate(ch):
                r = s.A.shape[1]
                self._planes_of[self._chunk_sites[ci][j]] = (dt, vbase, ubase, c0, r, ldq,
                                                            reg.view(ch[0].segments).n_rows)
                c0 += r

        # Problem tables, per activation dtype.
        # Tables are keyed by (dtype, rank blocks): one launch per key.
        pj: dict[tuple, _Table] = {}
        ft: dict[tuple, _Table] = {}
        pl = _Table(N.PL_FIELDS)
        fused_rows: list[tuple] = []
        stream_rows: dict[int, list[tuple]] = {}  # per rank-block count

        def tab(tables: dict, dt: torch.dtype, r: int, fields: int) -> _Table:
            return tables.setdefault((dt, (r + 15) // 16), _Table(fields))

        elem = {torch.bfloat16: 2, torch.float32: 4}
        for ci, (ch, (dt, rtot, rows_alloc, planes, vbase, ubase, ldq)) in enumerate(zip(chunks, chunk_layout)):
            qb = self.qbuf[dt]
            es = elem[dt]
            v = reg.view(ch[0].segments)
            n_rows, n_seg, valid, sf = v.n_rows, v.n_seg, v.valid, v.first

            def qaddr(base: int, row: int, qb=qb, ldq=ldq, es=es) -> int:
                return qb.data_ptr() + (base + row * ldq) * es

            x = ext[("lx", ci)]
            d_in = x.shape[1]
            # The seam's own V and U, when it kept them, become the planes
            # (odp_pack_planes); then one factor pass over X gives every
            # site's dA and one over each G its dB, and no activation or
            # output gradient is read twice.
            products = self._chunk_products[ci]
            if not products:
                # V = X [A_1 .. A_k]
                wx = wx_of[ci]
                if self._mirrored(ch, dt, v):
                    self._mirror_rows(ch[0], x, wx, ext[("lg", ci, 0)], ext[("lwb", ci, 0)], dt, v, qaddr, vbase,
                                      ubase, ldq, planes, es, pj, ft, tab, fused_rows, slot_base, stream_rows)
                    continue
                tab(pj, dt, rtot, N.PJ_FIELDS).add(
                    {
                        N.PJ_P: x.data_ptr(), N.PJ_LDP: x.stride(0), N.PJ_D: d_in,
                        N.PJ_W: wx.data_ptr(), N.PJ_R: rtot,
                        N.PJ_Q: qaddr(vbase, 0),
                        N.PJ_LDQ: ldq, N.PJ_NROWS: n_rows, N.PJ_SEG_FIRST: sf, N.PJ_NSEG: n_seg,
                    },
                    lib.odp_project_blocks(dtype_code(dt), _pj_rows(dt, v), rtot),
                    (valid * d_in + rtot * d_in + planes * rtot * valid) * es, 2 * valid * d_in * rtot,
                    io=valid * d_in * es,
                )
            c0 = 0
            a_leaves = []
            for j, s in enumerate(ch):
                r = s.A.shape[1]
                g = ext[("lg", ci, j)]
                wb = ext[("lwb", ci, j)]
                d_out = g.shape[1]
                if products:
                    for pkey, base in (("lv", vbase), ("lu", ubase)):
                        t = ext[(pkey, ci, j)]
                        pl.add({N.PL_SRC: t.data_ptr(), N.PL_LDS: t.stride(0), N.PL_R: r,
                                N.PL_DST: qaddr(base, c0), N.PL_LDQ: ldq, N.PL_NROWS: n_rows,
                                N.PL_SEG_FIRST: sf, N.PL_NSEG: n_seg, N.PL_DTYPE: dtype_code(dt)},
                               lib.odp_pack_planes_blocks(n_rows), (valid + n_rows) * r * es)
                if s.a_leaf is not None:
                    a_leaves.append((s.a_leaf, c0, r))
                # dB_i^T rows: pe[s][k][m] = scaling * sum_t V[k][t] G[t][m]
                frow = None
                if s.b_leaf is not None:
                    frow = {
                        N.FT_P: g.data_ptr(), N.FT_LDP: g.stride(0), N.FT_M: d_out,
                        N.FT_Q: qaddr(vbase, c0),
                        N.FT_LDQ: ldq, N.FT_R: r, N.FT_SEG_FIRST: sf, N.FT_NSEG: n_seg,
                        N.FT_SCALING: _f64_bits(s.scaling), N.FT_NLEAF: 1,
                        N.FT_LEAF0: pe_addr(s.b_leaf),
                        N.FT_LEAF0 + 1: 0 | (r << 16) | pe_bits(s.b_leaf),
                        N.FT_LEAF0 + 2: slot_base[s.b_leaf],
                    }
                if frow is not None and not products and self._fusable(dt, r, v, g):
                    # U and the dB rows in one pass over G, one workgroup per
                    # segment: a row per segment, so that the launch can run
                    # the longest first (the segment's pe rows start at its
                    # own offset).
                    frow.update({N.FP_W: wb.data_ptr(), N.FP_U: qaddr(ubase, c0), N.FT_NSEG: 1})
                    pe0 = pe_addr(s.b_leaf)
                    pe_es = self.pe[pe_dt[s.b_leaf]].element_size()
                    for j, ln in enumerate(v.segs.lengths):
                        row = dict(frow)
                        row[N.FT_SEG_FIRST] = sf + j
                        row[N.FT_LEAF0] = pe0 + j * r * d_out * pe_es
                        # G rows, the U/V planes and the dB rows of the segment;
                        # B itself is counted once per site.
                        fused_rows.append((-ln * d_out, len(fused_rows), row, 1,
                                           (ln * d_out + 2 * planes * r * ln) * es + r * d_out * es
                                           + (r * d_out * es if j == 0 else 0), ln * d_out * es,
                                           4 * ln * d_out * r))
                    c0 += r
                    continue
                if not products:
                    # U_i = G_i B_i^T into columns [c0, c0 + r) of the chunk's U planes.
                    tab(pj, dt, r, N.PJ_FIELDS).add(
                        {
                            N.PJ_P: g.data_ptr(), N.PJ_LDP: g.stride(0), N.PJ_D: d_out,
                            N.PJ_W: wb.data_ptr(), N.PJ_R: r,
                            N.PJ_Q: qaddr(ubase, c0),
                            N.PJ_LDQ: ldq, N.PJ_NROWS: n_rows, N.PJ_SEG_FIRST: sf, N.PJ_NSEG: n_seg,
                        },
                        lib.odp_project_blocks(dtype_code(dt), _pj_rows(dt, v), r),
                        (valid * d_out + r * d_out + planes * r * valid) * es, 2 * valid * d_out * r,
                        io=valid * d_out * es,
                    )
                if frow is not None and self._streamable(dt, [(0, r)], v, g):
                    self._stream_rows(frow, v, d_out, es, planes, stream_rows)
                elif frow is not None:
                    tab(ft, dt, r, N.FT_FIELDS).add(frow, n_seg * lib.odp_seg_factor_tiles(dtype_code(dt), d_out, r),
                                                    (valid * d_out + planes * r * valid) * es + n_seg * r * d_out * es,
                                                    2 * valid * d_out * r, io=valid * d_out * es)
                c0 += r
            if a_leaves:
                scal = {s.scaling for s in ch if s.a_leaf is not None}
                if len(scal) != 1:
                    # Different scalings cannot share one pass: split them.
                    for s_leaf, col0, r in a_leaves:
                        sc = next(s.scaling for s in ch if s.a_leaf == s_leaf)
                        arow = self._a_row(x, d_in, qaddr, ubase, col0, r, ldq, sf, n_seg, sc,
                                           [(s_leaf, col0, r)], pe_off, slot_base)
                        if self._streamable(dt, [(0, r)], v, x):
                            self._stream_rows(arow, v, d_in, es, planes, stream_rows)
                            continue
                        tab(ft, dt, r, N.FT_FIELDS).add(
                            arow, n_seg * lib.odp_seg_factor_tiles(dtype_code(dt), d_in, r),
                            (valid * d_in + planes * r * valid) * es + n_seg * r * d_in * es, 2 * valid * d_in * r,
                            io=valid * d_in * es)
                elif self._streamable(dt, [(c, rk) for _, c, rk in a_leaves], v, x) and (rtot + 15) // 16 <= 3:
                    # One leaf per 16-row block of U (q/k/v, gate/up at rank 16).
                    self._stream_rows(self._a_row(x, d_in, qaddr, ubase, 0, rtot, ldq, sf, n_seg, scal.pop(),
                                                  a_leaves, pe_off, slot_base),
                                      v, d_in, es, planes, stream_rows)
                else:
                    tab(ft, dt, rtot, N.FT_FIELDS).add(
                        self._a_row(x, d_in, qaddr, ubase, 0, rtot, ldq, sf, n_seg, scal.pop(),
                                    a_leaves, pe_off, slot_base),
                        n_seg * lib.odp_seg_factor_tiles(dtype_code(dt), d_in, rtot),
                        (valid * d_in + planes * rtot * valid) * es
                        + n_seg * sum(rk for _, _, rk in a_leaves) * d_in * es, 2 * valid * d_in * rtot,
                        io=valid * d_in * es)

        # Most work first (the fused launch has one workgroup per segment, of
        # very different lengths).
        fp = _Table(N.FT_FIELDS)
        for _, _, row, blocks, nbytes, io, fl in sorted(fused_rows, key=lambda t: (t[0], t[1])):
            fp.add(row, blocks, nbytes, fl, io=io)
        fst: dict[int, _Table] = {}
        for nkb in sorted(stream_rows):
            fst[nkb] = _Table(N.FT_FIELDS)
            for _, _, row, blocks, nbytes, io, fl in sorted(stream_rows[nkb], key=lambda t: (t[0], t[1])):
                fst[nkb].add(row, blocks, nbytes, fl, io=io)

        sq = _Table(N.SQ_FIELDS)
        mat_pe: dict[int, torch.Tensor] = {}
        for mi, m in enumerate(mats):
            pe_m = ext[("mat", mi)]
            v = leaf_view[m.leaf]
            n_seg = v.n_seg
            n = pe_m.shape[1]
            sq.add(
                {
                    N.SQ_X: pe_m.data_ptr(), N.SQ_N: n, N.SQ_NSEG: n_seg, N.SQ_SEG_FIRST: v.first,
                    N.SQ_SLOT: slot_base[m.leaf],
                    N.SQ_DTYPE: dtype_code(pe_m.dtype) | ((1 if self.square_f64 else 0) << 8)
                    | ((1 if self.raw_values else 0) << 9),
                },
                n_seg * lib.odp_sqnorm_blocks(n),
                n_seg * n * pe_m.element_size(), io=n_seg * n * pe_m.element_size(),
            )
            mat_pe[m.leaf] = pe_m

        self.lin_pe = torch.empty(pe_total, dtype=torch.bfloat16, device=dev)

        # Sites whose per-example gradients are not stored read X and G in
        # the Gram norm and the clipped-sum GEMM, which zero the feature
        # columns holding a non-finite value within each segment (so that the
        # result is nan_to_num of every per-example gradient).  One mask per
        # distinct tensor and segment list, found by odp_nonfinite_columns.
        # The same pass records each segment's largest finite |value| (one
        # uint32 per segment, zeroed at every run), from which the Gram and
        # GEMM kernels tell the segments whose products could overflow
        # float32; those take the outer form and the moments kernel, which
        # form M_s as the reference does.
        masks: dict[tuple, tuple[torch.Tensor, _SegView, int, int]] = {}
        mask_words = 0
        amax_words = 0

        def mask_of(t: torch.Tensor, v: _SegView) -> int:
            nonlocal mask_words, amax_words
            key = (t.data_ptr(), tuple(t.shape), tuple(t.stride()), v.first)
            if key not in masks:
                masks[key] = (t, v, mask_words, amax_words)
                mask_words += v.n_seg * ((t.shape[1] + 31) // 32)
                amax_words += v.n_seg
            return masks[key][2]

        def amax_of(t: torch.Tensor, v: _SegView) -> int:
            return self._amax.data_ptr() + 4 * masks[(t.data_ptr(), tuple(t.shape), tuple(t.stride()), v.first)][3]

        # With second moments, sites without stored gradients take the
        # moments kernel (odp_linear_moments), which forms each M_s tile and
        # zeroes its non-finite entries itself: only their Gram-form norms
        # read the masks.
        lin_mom = {i for i in range(len(lins)) if i not in lin_pe and self.second_moment}
        site_mask = {i: (mask_of(lin_x[i], lin_view[i]), mask_of(lin_g[i], lin_view[i]))
                     for i in range(len(lins))
                     if i not in lin_pe and (i not in lin_mom or lin_form[i] != N.FORM_OUTER)}
        self.nf_mask = torch.empty(max(mask_words, 1), dtype=torch.int32, device=dev)
        self._has_masks = mask_words > 0
        self._amax = torch.zeros(amax_words, dtype=torch.int32, device=dev)

        def mask_addr(w: int) -> int:
            return self.nf_mask.data_ptr() + 4 * w

        nft = _Table(N.NF_FIELDS)
        for t, v, off, aoff in masks.values():
            nft.add({N.NF_P: t.data_ptr(), N.NF_LDP: t.stride(0), N.NF_D: t.shape[1],
                     N.NF_SEG_FIRST: v.first, N.NF_NSEG: v.n_seg, N.NF_MASK: mask_addr(off),
                     N.NF_AMAX: self._amax.data_ptr() + 4 * aoff},
                    int(lib.odp_nonfinite_blocks(t.shape[1], v.n_seg)), v.valid * t.shape[1] * 2,
                    io=v.valid * t.shape[1] * 2)

        # Clipped sums read X' = c_i x_t (odp_linear_prescale) from a scratch
        # buffer, one X' per (activation, group, class), filled chunk by chunk
        # so that a chunk's X' fit in prescale_bytes; a site whose X' alone
        # does not fit scales its activations in registers instead.
        site_chunk: list[tuple[int, tuple] | None] = []
        xs_chunks: list[dict[tuple, tuple[int, int]]] = []
        cur: dict[tuple, tuple[int, int]] = {}
        cur_bytes = xs_bytes = 0
        for i, ls in enumerate(lins):
            if i in lin_pe or i in lin_mom:
                site_chunk.append(None)
                continue
            x, lf = lin_x[i], self.leaves[ls.w_leaf]
            nbytes = -(-x.shape[0] * x.shape[1] * 2 // 256) * 256
            if nbytes > self._prescale_budget:
                site_chunk.append(None)
                continue
            k = (x.data_ptr(), tuple(x.shape), tuple(x.stride()), lin_view[i].first, lf.group, lf.cls)
            if k not in cur:
                if cur_bytes + nbytes > self._prescale_budget:
                    xs_chunks.append(cur)
                    cur, cur_bytes = {}, 0
                cur[k] = (cur_bytes // 2, i)
                cur_bytes += nbytes
                xs_bytes = max(xs_bytes, cur_bytes)
            site_chunk.append((len(xs_chunks), k))
        if cur:
            xs_chunks.append(cur)
        self.xs = torch.empty(xs_bytes // 2, dtype=torch.bfloat16, device=dev)
        xs_pre = [_Table(N.LN_FIELDS) for _ in xs_chunks]
        xs_sum = [_Table(N.LN_FIELDS) for _ in xs_chunks]
        for c, members in enumerate(xs_chunks):
            for off, i in members.values():
                x, v, lf = lin_x[i], lin_view[i], self.leaves[lins[i].w_leaf]
                xs_pre[c].add({N.LN_X: x.data_ptr(), N.LN_LDX: x.stride(0), N.LN_DIN: x.shape[1],
                               N.LN_SEG_FIRST: v.first, N.LN_NSEG: v.n_seg, N.LN_NROWS: x.shape[0],
                               N.LN_FLAGS: (lf.group << 8) | (lf.cls << 24), N.LN_OUT: self.xs[off:].data_ptr(),
                               N.LN_XMASK: mask_addr(site_mask[i][0])},
                              int(lib.odp_linear_prescale_blocks(x.shape[0])), 2 * v.valid * x.shape[1] * 2,
                              io=v.valid * x.shape[1] * 2)
        lnt = {N.FORM_OUTER: _Table(N.LN_FIELDS), N.FORM_GRAM: _Table(N.LN_FIELDS),
               N.FORM_GRAM256: _Table(N.LN_FIELDS)}
        lng = _Table(N.LN_FIELDS)  # guarded outer-form norms of Gram sites
        lmg = _Table(N.LN_FIELDS)  # guarded moments (first moment) of clipped-sum GEMM sites
        # fp32 scratch of the 256-row-block Gram kernel (its X blocks).
        self.gram_scr = (torch.empty(scr_total // 4, dtype=torch.float32, device=dev) if scr_total
                         else None)
        lsum = _Table(N.LN_FIELDS)
        lmom = _Table(N.LN_FIELDS)
        for i, ls in enumerate(lins):
            x, g = lin_x[i], lin_g[i]
            d_in, d_out = x.shape[1], g.shape[1]
            form = lin_form[i]
            v = lin_view[i]
            n_seg, valid = v.n_seg, v.valid
            common = {
                N.LN_X: x.data_ptr(), N.LN_LDX: x.stride(0), N.LN_G: g.data_ptr(), N.LN_LDG: g.stride(0),
                N.LN_DIN: d_in, N.LN_DOUT: d_out, N.LN_SEG_FIRST: v.first, N.LN_NSEG: n_seg,
            }
            if i in site_mask:
                common[N.LN_XMASK] = mask_addr(site_mask[i][0])
                common[N.LN_GMASK] = mask_addr(site_mask[i][1])
                common[N.LN_XAMAX] = amax_of(x, v)
                common[N.LN_GAMAX] = amax_of(g, v)
            if form in (N.FORM_GRAM, N.FORM_GRAM256):
                fl = sum(ln * ln for ln in v.segs.lengths) * (d_in + d_out)
            else:
                fl = 2 * valid * d_in * d_out
            blocks = int(lib.odp_linear_norm_blocks(form, d_in, d_out, v.max_len, n_seg))
            nb_max = (v.max_len + 255) // 256 if form == N.FORM_GRAM256 else (v.max_len + 127) // 128
            pe_at = self.lin_pe[lin_pe[i]:].data_ptr() if i in lin_pe else 0
            scr_at = self.gram_scr.data_ptr() + lin_scr[i] if i in lin_scr else 0
            lnt[form].add({**common, N.LN_SLOT: slot_base[ls.w_leaf] + lin_off[i], N.LN_NB: nb_max,
                           N.LN_PE: pe_at, N.LN_NFFLAG: self._nf_flag_addr, N.LN_SCRATCH: scr_at}, blocks,
                          valid * (d_in + d_out) * 2 + (n_seg * d_in * d_out * 2 if pe_at else 0), fl,
                          io=valid * (d_in + d_out) * 2)
            if i in lin_goff:
                lng.add({**common, N.LN_SLOT: slot_base[ls.w_leaf] + lin_goff[i], N.LN_NFFLAG: self._nf_flag_addr},
                        int(lib.odp_linear_norm_blocks(N.FORM_OUTER_GUARDED, d_in, d_out, v.max_len, n_seg)))
            if i in lin_pe:
                continue
            lf = self.leaves[ls.w_leaf]
            out = self.out[ls.w_leaf] if ls.index is None else self.out[ls.w_leaf][ls.index]
            flags = dtype_code(lf.out_dtype) | (lf.group << 8) | (lf.cls << 24)
            if i in lin_mom:
                o2 = self.out2[ls.w_leaf] if ls.index is None else self.out2[ls.w_leaf][ls.index]
                lmom.add({**common, N.LN_OUT: out.data_ptr(), N.LN_OUT2: o2.data_ptr(), N.LN_FLAGS: flags},
                         int(lib.odp_linear_moments_blocks(d_in, d_out, 0)),
                         valid * (d_in + d_out) * 2 + 2 * d_in * d_out * out.element_size(),
                         2 * valid * d_in * d_out,
                         io=valid * (d_in + d_out) * 2 + 2 * d_in * d_out * out.element_size())
                continue
            row, into = {**common, N.LN_OUT: out.data_ptr(), N.LN_FLAGS: flags}, lsum
            # The same output, written only if a segment is at risk of
            # float32 overflow (the GEMM then skips the site).
            lmg.add({**common, N.LN_OUT: out.data_ptr(), N.LN_OUT2: 0, N.LN_FLAGS: flags},
                    int(lib.odp_linear_moments_blocks(d_in, d_out, 1)))
            if site_chunk[i] is not None:
                c, k = site_chunk[i]
                row[N.LN_X] = self.xs[xs_chunks[c][k][0]:].data_ptr()
                row[N.LN_LDX] = d_in
                into = xs_sum[c]
            into.add(row, int(lib.odp_linear_sum_blocks(d_in, d_out)),
                     valid * (d_in + d_out) * 2 + d_in * d_out * out.element_size(),
                     2 * valid * d_in * d_out,
                     io=(0 if site_chunk[i] is not None else valid * (d_in + d_out) * 2)
                     + d_in * d_out * out.element_size())
        lin_leaves = {ls.w_leaf for ls in lins}

        ss = _Table(N.SS_FIELDS)
        for i, off in lin_pe.items():
            ls, v = lins[i], lin_view[i]
            lf = self.leaves[ls.w_leaf]
            out = self.out[ls.w_leaf] if ls.index is None else self.out[ls.w_leaf][ls.index]
            out2 = 0
            if self.out2 is not None:
                o2 = self.out2[ls.w_leaf]
                out2 = (o2 if ls.index is None else o2[ls.index]).data_ptr()
            M = ls.x.shape[-1] * ls.g.shape[-1]
            flags = (dtype_code(lf.out_dtype) | (lf.group << 16) | (lf.cls << 40) | (int(self.sum_f64) << 48)
                     | (N.DTYPE_BF16 << 56))
            ss.add({N.SS_PE: self.lin_pe[off:].data_ptr(), N.SS_M: M, N.SS_RANK: 1, N.SS_SEG_FIRST: v.first,
                    N.SS_NSEG: v.n_seg, N.SS_OUT: out.data_ptr(), N.SS_FLAGS: flags, N.SS_OUT2: out2},
                   lib.odp_scale_sum_blocks(M),
                   v.n_seg * M * 2 + M * out.element_size() * (2 if self.out2 is not None else 1),
                   io=M * out.element_size() * (2 if self.out2 is not None else 1))
        for i, lf in enumerate(self.leaves):
            if i in lin_leaves:
                continue
            out = self.out[i]
            out2 = self.out2[i].data_ptr() if self.out2 is not None else 0
            v = leaf_view[i]
            n_seg = v.n_seg
            if i in mat_pe:
                pe_m = mat_pe[i]
                rank, M, transpose, pdt, pe_a = 1, pe_m.shape[1], 0, dtype_code(pe_m.dtype), pe_m.data_ptr()
            else:
                rank, M = leaf_rank_m[i]
                transpose = 1 if self._leaf_transposed(i, sites) else 0
                pdt, pe_a = dtype_code(pe_dt[i]), pe_addr(i)
            flags = (dtype_code(lf.out_dtype) | (transpose << 8) | (lf.group << 16) | (lf.cls << 40)
                     | (int(self.sum_f64) << 48) | (int(self.raw_values and i in mat_pe) << 52) | (pdt << 56))
            ss.add(
                {
                    N.SS_PE: pe_a, N.SS_M: M, N.SS_RANK: rank, N.SS_SEG_FIRST: v.first,
                    N.SS_NSEG: n_seg, N.SS_OUT: out.data_ptr(), N.SS_FLAGS: flags, N.SS_OUT2: out2,
                },
                lib.odp_scale_sum_blocks(rank * M),
                n_seg * rank * M * (self.pe[pe_dt[i]].element_size() if i not in mat_pe else mat_pe[i].element_size())
                + rank * M * out.element_size() * (2 if self.out2 is not None else 1),
                io=rank * M * out.element_size() * (2 if self.out2 is not None else 1),
            )

        # Upload everything in one copy.
        pack = _Pack()
        idx = {}
        seg_st, seg_ln, seg_ex = reg.arrays()
        idx["seg_start"] = pack.add(seg_st)
        idx["seg_len"] = pack.add(seg_ln)
        idx["seg_ex"] = pack.add(seg_ex)
        self._launch: list[tuple] = []
        tabs = [("pack", None, pft), ("planes", None, pl)]
        for key in sorted(pj, key=lambda k: (str(k[0]), k[1])):
            tabs.append(("project", key, pj[key]))
        tabs.append(("factor_project", None, fp))
        for nkb in sorted(fst):
            tabs.append(("factor_stream", nkb, fst[nkb]))
        for key in sorted(ft, key=lambda k: (str(k[0]), k[1])):
            tabs.append(("factor", key, ft[key]))
        tabs.append(("sqnorm", None, sq))
        tabs.append(("nonfinite", None, nft))
        tabs.append(("lin_norm", N.FORM_OUTER, lnt[N.FORM_OUTER]))
        tabs.append(("lin_norm", N.FORM_GRAM, lnt[N.FORM_GRAM]))
        tabs.append(("lin_norm", N.FORM_GRAM256, lnt[N.FORM_GRAM256]))
        tabs.append(("lin_norm", N.FORM_OUTER_GUARDED, lng))
        tabs.append(("scale_sum", None, ss))
        for c in range(len(xs_chunks)):
            tabs.append(("lin_prescale", c, xs_pre[c]))
            tabs.append(("lin_sum", c, xs_sum[c]))
        tabs.append(("lin_sum", None, lsum))
        tabs.append(("lin_moments", None, lmom))
        tabs.append(("lin_moments", 1, lmg))
        tab_idx = []
        for name, dt, t in tabs:
            probs, ws, total = t.arrays()
            tab_idx.append((name, dt, pack.add(probs), pack.add(ws), len(t.rows), total,
                            (t.nbytes, t.nflops, t.io_bytes)))
        idx["gstart"] = pack.add(gstart)
        idx["thr"] = pack.add(np.asarray(self.clip.thresholds, dtype=np.float64))
        guards = self.clip.guards or [(1.0, 0.0, torch.float32)]
        idx["guard"] = pack.add(np.asarray([[g[0], g[1]] for g in guards], dtype=np.float64).reshape(-1))
        idx["cls_dt"] = pack.add(np.asarray([dtype_code(g[2]) for g in guards], dtype=np.int32))
        views = pack.upload(dev)
        self._views = views
        self._pack = pack
        self._thr_idx, self._guard_idx = idx["thr"], idx["guard"]
        # ext now also holds the output buffers, after the inputs' tensors.
        patch_keys, patches = self._pointer_fields([pack.array(pi) for _, _, pi, _, _, _, _ in tab_idx], ext)
        pos = {k: i for i, k in enumerate(ext)}
        src_pos = np.asarray([pos[k] for k in patch_keys], dtype=np.int64)
        self._patches = [(vals, sel, src_pos[kidx], off) for vals, sel, kidx, off in patches]
        self._stream_id = _stream()
        self.seg_start, self.seg_len, self.seg_ex = (views[idx[k]] for k in ("seg_start", "seg_len", "seg_ex"))
        self.gstart, self.thr = views[idx["gstart"]], views[idx["thr"]]
        self.guard, self.cls_dt = views[idx["guard"]], views[idx["cls_dt"]]
        self.tables = [(name, dt, views[pi], views[wi], n, total) for name, dt, pi, wi, n, total, _ in tab_idx]
        # Per launch, in launch order: (stage, key, workgroups, algorithmic bytes, algorithmic flops,
        # contract bytes: the part of the bytes that reads activations and
        # output gradients or writes the clipped sums).
        info = [(name, dt, total, nb[0], nb[1], nb[2]) for name, dt, _, _, _, total, nb in tab_idx if total > 0]
        after_clip = _AFTER_CLIP
        self.launch_info = [i for i in info if i[0] not in after_clip] + [i for i in info if i[0] in after_clip]

    @staticmethod
    def _pointer_fields(arrays: list[np.ndarray], ext: dict[tuple, torch.Tensor]) -> tuple[list, list[tuple]]:
        """Every table field that holds an address inside one of the tensors of
        `ext`: the keys of those tensors, and per array that has such fields
        (flat view, field indices, key indices, byte offsets into the tensor)."""
        keys, lo, hi = [], [], []
        for k, t in ext.items():
            if t.numel() == 0:
                continue
            extent = 1 + sum((n - 1) * st for n, st in zip(t.shape, t.stride()))
            keys.append(k)
            lo.append(t.data_ptr())
            hi.append(t.data_ptr() + extent * t.element_size())
        order = np.argsort(np.asarray(lo, dtype=np.int64), kind="stable")
        lo_s = np.asarray(lo, dtype=np.int64)[order]
        hi_s = np.asarray(hi, dtype=np.int64)[order]
        out = []
        for arr in arrays:
            vals = arr.reshape(-1)
            pos = np.searchsorted(lo_s, vals, side="right") - 1
            ok = (pos >= 0) & (vals < hi_s[np.maximum(pos, 0)])
            sel = np.nonzero(ok)[0]
            if sel.size:
                out.append((vals, sel, order[pos[sel]], vals[sel] - lo_s[pos[sel]]))
        return keys, out

    def rebind(self, lora_sites: list[LoraSite] = (), materialized: list[MaterializedLeaf] = (),
               linear_sites: list[LinearSite] = (), clip: ClipSpec | None = None, key: tuple | None = None,
               lora_ptrs: torch.Tensor | None = None) -> bool:
        """Points the plan at a new call's inputs with the same structure and
        gives it fresh outputs; scratch buffers and tables are reused.

        The caller guarantees the structure (the same sites, leaf layout and
        segments in the same order).  With ``key``, the new inputs' plan_key,
        equal to the plan's own, shapes, strides, dtypes, devices, alignment
        and activation sharing are known to match; without it the tensors
        derived from the new inputs are checked to lay out like the ones the
        plan was built from.  Returns False (and leaves the plan unusable)
        when they do not, or when the current stream is not the one the plan
        ran on (its scratch is ordered on that stream).  ``lora_ptrs``: the
        LoRA sites' addresses that plan_key wrote while computing ``key``;
        with them the LoRA side is re-pointed without reading the site
        tensors again.
        """
        if _stream() != self._stream_id:
            return False
        sites, mats, lins = lora_sites, list(materialized), list(linear_sites)
        if clip is not None and (len(clip.thresholds) != self.n_groups or clip.mode != self.clip.mode
                                 or len(clip.guards) != len(self.clip.guards)):
            return False
        trusted = key is not None and key == self.key
        fast = self._fast if trusted and lora_ptrs is not None else None
        chunks = []
        if fast is None:
            try:
                chunks = [[sites[k] for k in idx] for idx in self._chunk_sites]
            except IndexError:
                return False
        if not trusted:
            # The sites of a chunk read one activation (the plan projects it once).
            for ci, ch in enumerate(chunks):
                x0 = ch[0].x
                for s in ch[1:]:
                    if s.x.data_ptr() != x0.data_ptr() or s.x.shape != x0.shape or s.x.stride() != x0.stride():
                        return False
                # A chunk planned on the seam's V and U needs them again.
                if self._chunk_products[ci] and not uses_seam_products(ch):
                    return False
        if fast is not None:
            src, n_lora = fast
            outs = list(self._alloc_outputs().values())
            tail = self._other_external(mats, lins, self._direct, n_lora) + outs
            ptr = np.empty(len(self._ext_keys) + len(outs), dtype=np.int64)
            ptr[:n_lora] = lora_ptrs.numpy()[src[:n_lora]]
            ptr[n_lora:] = np.fromiter((t.data_ptr() for t in tail), dtype=np.int64, count=len(tail))
            tensors = tail
        else:
            tensors = self._external_list(chunks, mats, lins, self._direct if trusted else None)
            if not trusted and _layout(dict(zip(self._ext_keys, tensors))) != self._layout_in:
                return False
            tensors += self._alloc_outputs().values()
            ptr = np.fromiter((t.data_ptr() for t in tensors), dtype=np.int64, count=len(tensors))
        for vals, sel, pos, off in self._patches:
            vals[sel] = ptr[pos] + off
        if clip is not None:
            self.clip = clip
            self._pack.array(self._thr_idx)[:] = np.asarray(clip.thresholds, dtype=np.float64)
            guards = clip.guards or [(1.0, 0.0, torch.float32)]
            self._pack.array(self._guard_idx)[:] = np.asarray([[g[0], g[1]] for g in guards],
                                                              dtype=np.float64).reshape(-1)
        self._ext = tensors  # kept alive while the plan points at them
        self._pack.refresh()
        return True

    def _ext_sources(self, chunks: list[list[LoraSite]], mats: list[MaterializedLeaf],
                     lins: list[LinearSite]) -> dict[tuple, torch.Tensor]:
        """The input tensor each external tensor derives from."""
        src: dict[tuple, torch.Tensor] = {}
        for ci, ch in enumerate(chunks):
            src[("lx", ci)] = ch[0].x
            for j, s in enumerate(ch):
                src[("lg", ci, j)] = s.g
                src[("lwb", ci, j)] = s.B
                src[("la", ci, j)] = s.A
                if self._chunk_products[ci]:
                    src[("lv", ci, j)] = s.v
                    src[("lu", ci, j)] = s.u
        for mi, m in enumerate(mats):
            src[("mat", mi)] = m.per_example
        for i, ls in enumerate(lins):
            src[("linx", i)] = ls.x
            src[("ling", i)] = ls.g
        return src

    def _fast_map(self, chunks: list[list[LoraSite]], ext: dict[tuple, torch.Tensor], n_sites: int):
        """Where rebind's fast path finds each LoRA input address: when every
        LoRA input is read in place, the address of ("lx", c), ("lg", c, j),
        ("lwb", c, j), ("la", c, j), ("lv", c, j) and ("lu", c, j) is the
        caller's x, g, B, A, v or u (entry LORA_PTRS site + 0, 1, 3, 2, 4 or
        5 of the host helper's address list).  None when some input was
        copied at build time, or without the helper."""
        if _host.load() is None or not chunks:
            return None
        slot = {"lx": 0, "lg": 1, "la": 2, "lwb": 3, "lv": 4, "lu": 5}
        keys = self._ext_keys
        src = np.full(len(keys), -1, dtype=np.int64)
        n_lora = 0
        for p, k in enumerate(keys):
            kind = k[0]
            if kind not in slot:
                continue
            n_lora += 1
            ci = k[1]
            j = 0 if kind == "lx" else k[2]
            s = chunks[ci][j]
            t = (s.x, s.g, s.A, s.B, s.v, s.u)[slot[kind]]
            if ext[k].data_ptr() != t.data_ptr():
                return None
            src[p] = LORA_PTRS * self._chunk_sites[ci][j] + slot[kind]
        return src, n_lora

    @staticmethod
    def _factor_groups(chunks: list[list[LoraSite]], products: list[bool]) -> list[list[int]]:
        """Chunks whose stacked A^T come out of one copy: same dtype and d_in
        (chunks that read the seam's V and U project nothing and need none)."""
        by_width: dict[tuple, list[int]] = {}
        for ci, ch in enumerate(chunks):
            if not products[ci]:
                by_width.setdefault((ch[0].x.dtype, ch[0].A.shape[0]), []).append(ci)
        return list(by_width.values())

    def _external_keys(self, chunks: list[list[LoraSite]], n_mats: int, n_lins: int) -> list[tuple]:
        """Keys of the tensors _external_list returns, in its order: per LoRA
        chunk its activation rows ("lx", c) and per site of the chunk its
        output gradient rows ("lg", c, j), B ("lwb", c, j) and A ("la", c, j)
        (and the seam's V ("lv", c, j) and U ("lu", c, j) rows when it uses them);
        materialised leaves ("mat", m) as [n_seg, n]; linear sites' rows
        ("linx", i), ("ling", i)."""
        keys = []
        for ci, ch in enumerate(chunks):
            keys.append(("lx", ci))
            for j in range(len(ch)):
                keys += [("lg", ci, j), ("lwb", ci, j), ("la", ci, j)]
                if self._chunk_products[ci]:
                    keys += [("lv", ci, j), ("lu", ci, j)]
        keys += [("mat", mi) for mi in range(n_mats)]
        for i in range(n_lins):
            keys += [("linx", i), ("ling", i)]
        return keys

    def _external_list(self, chunks: list[list[LoraSite]], mats: list[MaterializedLeaf],
                       lins: list[LinearSite], direct: list[bool] | None = None) -> list[torch.Tensor]:
        """The tensors the tables point to that come from the caller's inputs
        (keys from _external_keys).  Where ``direct`` is set the input tensor
        itself stands in for its row view."""
        out: list[torch.Tensor] = []
        p = 0
        with torch.no_grad():
            for ci, ch in enumerate(chunks):
                dt = ch[0].x.dtype
                x = ch[0].x
                out.append(x if direct and direct[p] else _rows(x))
                p += 1
                for s in ch:
                    out.append(s.g if direct and direct[p] else _rows(s.g))
                    b = s.B
                    out.append(b if b.dtype == dt and b.is_contiguous() else b.to(dt).contiguous())
                    out.append(s.A)  # read in place by odp_pack_factors
                    p += 3
                    if self._chunk_products[ci]:
                        out.append(s.v if direct and direct[p] else _seam_rows(s.v))
                        out.append(s.u if direct and direct[p + 1] else _seam_rows(s.u))
                        p += 2
        return out + self._other_external(mats, lins, direct, p)

    def _other_external(self, mats: list[MaterializedLeaf], lins: list[LinearSite], direct: list[bool] | None,
                        p: int) -> list[torch.Tensor]:
        """_external_list's materialised and linear-site tensors (from position p)."""
        out: list[torch.Tensor] = []
        for m in mats:
            if direct and direct[p]:
                out.append(m.per_example)
            else:
                pe_m = m.per_example.detach()
                if pe_m.dtype not in _DTYPE_CODE:
                    pe_m = pe_m.float()
                out.append(pe_m.reshape(pe_m.shape[0], -1).contiguous())
            p += 1
        for ls in lins:
            out.append(ls.x if direct and direct[p] else _rows(ls.x))
            out.append(ls.g if direct and direct[p + 1] else _rows(ls.g))
            p += 2
        return out

    def _alloc_outputs(self) -> dict[tuple, torch.Tensor]:
        """Fresh output buffers: one flat buffer per output dtype (and one more
        for the second moments), the per-example results, and the leaves as
        views of the flat buffers.  Returns the buffers the tables point into."""
        dev = self.device
        if not hasattr(self, "_out_groups"):
            self._plan_out_layout()
        self.flat = {dt: torch.empty(max(n, 1), dtype=dt, device=dev) for dt, n in self._out_sizes.items()}
        self.out: list[torch.Tensor] = self._leaf_views(self.flat)
        self.out2: list[torch.Tensor] | None = None
        outs = {("flat", str(dt)): t for dt, t in self.flat.items()}
        if self.second_moment:
            flat2 = {dt: torch.empty(max(n, 1), dtype=dt, device=dev) for dt, n in self._out_sizes.items()}
            self.out2 = self._leaf_views(flat2)
            outs.update({("flat2", str(dt)): t for dt, t in flat2.items()})
        # The per-example results, carved from one allocation (each part
        # 256-byte aligned).
        if not hasattr(self, "_res_parts"):
            G, C, E = self.n_groups, self.n_cls, self.segments.n_ex
            parts = [((C, G, E), torch.float64), ((E,), torch.float32), ((G, E), torch.float32),
                     ((G, E), torch.uint8), ((E,), torch.uint8)]
            offs, total = [], 0
            for shape, dt in parts:
                offs.append(total)
                total += (math.prod(shape) * dt.itemsize + 255) // 256 * 256
            self._res_parts = (parts, offs, total)
            host = _host.load()
            self._res_maker = None if host is None else host.ViewMaker(
                [0] * len(parts), [list(sh) for sh, _ in parts],
                [[math.prod(sh[i + 1 :]) for i in range(len(sh))] for sh, _ in parts],
                [o // dt.itemsize for o, (_, dt) in zip(offs, parts)],
                [torch.empty(0, dtype=dt) for _, dt in parts])
        parts, offs, total = self._res_parts
        buf = torch.empty(total, dtype=torch.uint8, device=dev)
        if self._res_maker is not None:
            self.scales, self.norms, self.group_norms, self.clipped, self.clipped_total = self._res_maker.make([buf])
        else:
            self.scales, self.norms, self.group_norms, self.clipped, self.clipped_total = (
                buf[o : o + math.prod(shape) * dt.itemsize].view(dt).view(shape)
                for o, (shape, dt) in zip(offs, parts))
        return outs

    def _plan_out_layout(self) -> None:
        """Where each leaf lives in its dtype's flat buffer: leaves of one shape
        back to back, each padded to a multiple of 64 elements (so that every
        leaf starts 128-byte aligned), groups in order of first appearance."""
        groups: dict[tuple, list[int]] = {}
        for i, lf in enumerate(self.leaves):
            groups.setdefault((lf.out_dtype, tuple(lf.shape)), []).append(i)
        sizes: dict[torch.dtype, int] = {}
        self._out_groups = []  # (dtype, offset, count, padded size, size, shape)
        order = []
        for (dt, shape), idx in groups.items():
            n = math.prod(shape)
            padded = (n + 63) // 64 * 64
            off = sizes.get(dt, 0)
            self._out_groups.append((dt, off, len(idx), padded, n, shape))
            sizes[dt] = off + len(idx) * padded
            order += idx
        self._out_sizes = sizes
        self._out_perm = [0] * len(order)
        for pos, i in enumerate(order):
            self._out_perm[i] = pos
        # The same views made by the host helper in one call, when it is built.
        self._views_maker = None
        host = _host.load()
        if host is not None:
            buf_of = {dt: i for i, dt in enumerate(sizes)}
            where = {}
            for dt, off, k, padded, n, shape in self._out_groups:
                for j in range(k):
                    where[len(where)] = (buf_of[dt], off + j * padded, shape)
            bufs, shapes, strides, offs = [], [], [], []
            for i in range(len(self.leaves)):
                b, o, shape = where[self._out_perm[i]]
                st, acc = [], 1
                for d in reversed(shape):
                    st.append(acc)
                    acc *= d
                bufs.append(b)
                shapes.append(list(shape))
                strides.append(list(reversed(st)))
                offs.append(o)
            self._views_maker = host.ViewMaker(bufs, shapes, strides, offs)

    def _leaf_views(self, flat: dict[torch.dtype, torch.Tensor]) -> list[torch.Tensor]:
        if self._views_maker is not None:
            return self._views_maker.make([flat[dt] for dt in self._out_sizes])
        views: list[torch.Tensor] = []
        for dt, off, k, padded, n, shape in self._out_groups:
            block = flat[dt][off : off + k * padded].view(k, padded)
            if n != padded:
                block = block[:, :n]
            views.extend(block.view(k, *shape).unbind(0))
        return [views[p] for p in self._out_perm]

    def _mirrored(self, ch: list[LoraSite], dt: torch.dtype, v: _SegView) -> bool:
        """Whether a one-site chunk reads its activation once and its output
        gradient twice (U = G B^T first, then V and dA in one fused pass over
        X, then dB): fewer bytes when d_in > d_out, e.g. a down projection."""
        if len(ch) != 1 or ch[0].a_leaf is None:
            return False
        s = ch[0]
        x = _rows(s.x)
        return x.shape[1] > s.g.shape[-1] and self._fusable(dt, s.A.shape[1], v, x)

    def _mirror_rows(self, s, x, wx, g, wb, dt, v, qaddr, vbase, ubase, ldq, planes, es, pj, ft, tab, fused_rows,
                     slot_base, stream_rows) -> None:
        lib = N.load()
        r = s.A.shape[1]
        d_in = x.shape[1]
        d_out = g.shape[1]
        n_rows, n_seg, valid, sf = v.n_rows, v.n_seg, v.valid, v.first
        # U = G B^T (the projection kernel on G).
        tab(pj, dt, r, N.PJ_FIELDS).add(
            {
                N.PJ_P: g.data_ptr(), N.PJ_LDP: g.stride(0), N.PJ_D: d_out,
                N.PJ_W: wb.data_ptr(), N.PJ_R: r,
                N.PJ_Q: qaddr(ubase, 0),
                N.PJ_LDQ: ldq, N.PJ_NROWS: n_rows, N.PJ_SEG_FIRST: sf, N.PJ_NSEG: n_seg,
            },
            lib.odp_project_blocks(dtype_code(dt), _pj_rows(dt, v), r),
            (valid * d_out + r * d_out + planes * r * valid) * es, 2 * valid * d_out * r, io=valid * d_out * es,
        )
        # V = X A and the dA^T rows (scaling * sum_t U[k][t] X[t][m]) in one
        # pass over X: the fused kernel with X, A^T and U in the places of G,
        # B and V.  One row per segment, most work first.
        pe0 = self._pe_addr(s.a_leaf)
        pe_es = self.pe[dt].element_size()
        row = {
            N.FT_P: x.data_ptr(), N.FT_LDP: x.stride(0), N.FT_M: d_in,
            N.FT_Q: qaddr(ubase, 0),
            N.FT_LDQ: ldq, N.FT_R: r, N.FT_NSEG: 1,
            N.FT_SCALING: _f64_bits(s.scaling), N.FT_NLEAF: 1,
            N.FT_LEAF0 + 1: 0 | (r << 16) | self._pe_bits(s.a_leaf),
            N.FT_LEAF0 + 2: slot_base[s.a_leaf],
            N.FP_W: wx.data_ptr(), N.FP_U: qaddr(vbase, 0),
        }
        for j, ln in enumerate(v.segs.lengths):
            rj = dict(row)
            rj[N.FT_SEG_FIRST] = sf + j
            rj[N.FT_LEAF0] = pe0 + j * r * d_in * pe_es
            fused_rows.append((-ln * d_in, len(fused_rows), rj, 1,
                               (ln * d_in + 2 * planes * r * ln) * es + r * d_in * es
                               + (r * d_in * es if j == 0 else 0), ln * d_in * es, 4 * ln * d_in * r))
        # dB^T rows from G and V.
        if s.b_leaf is not None:
            brow = {
                N.FT_P: g.data_ptr(), N.FT_LDP: g.stride(0), N.FT_M: d_out,
                N.FT_Q: qaddr(vbase, 0),
                N.FT_LDQ: ldq, N.FT_R: r, N.FT_SEG_FIRST: sf, N.FT_NSEG: n_seg,
                N.FT_SCALING: _f64_bits(s.scaling), N.FT_NLEAF: 1,
                N.FT_LEAF0: self._pe_addr(s.b_leaf),
                N.FT_LEAF0 + 1: 0 | (r << 16) | self._pe_bits(s.b_leaf),
                N.FT_LEAF0 + 2: slot_base[s.b_leaf],
            }
            if self._streamable(dt, [(0, r)], v, g):
                self._stream_rows(brow, v, d_out, es, planes, stream_rows)
            else:
                tab(ft, dt, r, N.FT_FIELDS).add(
                    brow, n_seg * lib.odp_seg_factor_tiles(dtype_code(dt), d_out, r),
                    (valid * d_out + planes * r * valid) * es + n_seg * r * d_out * es, 2 * valid * d_out * r,
                    io=valid * d_out * es)

    def _fusable(self, dt: torch.dtype, r: int, v: _SegView, g: torch.Tensor) -> bool:
        """Whether a site's G side runs as one odp_seg_factor_project pass."""
        if not self.fuse_g_side or dt != torch.bfloat16 or r > 16:
            return False
        lib = N.load()
        return v.max_len <= lib.odp_factor_project_max_len() and v.max_len * g.stride(0) * 2 < 2**31

    def _streamable(self, dt: torch.dtype, leaves: list[tuple[int, int]], v: _SegView, p: torch.Tensor) -> bool:
        """Whether a factor problem over P whose leaves sit at these (column
        in Q, rank) pairs runs as odp_seg_factor_stream: bf16, every leaf on
        a 16-row block of its own, segments within the kernel's length."""
        if not self.stream_factors or dt != torch.bfloat16:
            return False
        if not leaves or any(c % 16 or rk > 16 for c, rk in leaves):
            return False
        lib = N.load()
        return v.max_len <= lib.odp_factor_project_max_len() and v.max_len * p.stride(0) * 2 < 2**31

    def _stream_rows(self, row: dict, v: _SegView, M: int, es: int, planes: int, out: dict) -> None:
        """A factor problem as odp_seg_factor_stream rows: one per segment,
        each leaf's pe rows at the segment's own offset, so that the launch
        can run the most work per workgroup first."""
        lib = N.load()
        r = int(row[N.FT_R])
        pe_es = self.pe[torch.bfloat16].element_size()
        groups = int(lib.odp_seg_factor_stream_groups(M))
        ranks = [(row[N.FT_LEAF0 + 3 * li + 1] >> 16) & 0xFFFF for li in range(int(row[N.FT_NLEAF]))]
        lst = out.setdefault((r + 15) // 16, [])
        for j, ln in enumerate(v.segs.lengths):
            rj = dict(row)
            rj[N.FT_SEG_FIRST] = v.first + j
            rj[N.FT_NSEG] = 1
            for li, rk in enumerate(ranks):
                rj[N.FT_LEAF0 + 3 * li] = row[N.FT_LEAF0 + 3 * li] + j * rk * M * pe_es
            rj[N.FT_GROUPS] = groups
            lst.append((-ln * M / groups, len(lst), rj, groups,
                        (ln * M + planes * r * ln) * es + sum(ranks) * M * es, ln * M * es, 2 * ln * M * r))

    def _a_row(self, x, d_in, qaddr, ubase, col0, r, ldq, seg_first, n_seg, scaling, leaves, pe_off, slot_base):
        row = {
            N.FT_P: x.data_ptr(), N.FT_LDP: x.stride(0), N.FT_M: d_in,
            N.FT_Q: qaddr(ubase, col0),
            N.FT_LDQ: ldq, N.FT_R: r, N.FT_SEG_FIRST: seg_first, N.FT_NSEG: n_seg,
            N.FT_SCALING: _f64_bits(scaling), N.FT_NLEAF: len(leaves),
        }
        for li, (leaf, c, rk) in enumerate(sorted(leaves, key=lambda t: t[1])):
            row[N.FT_LEAF0 + 3 * li] = self._pe_addr(leaf)
            row[N.FT_LEAF0 + 3 * li + 1] = (c - col0) | (rk << 16) | self._pe_bits(leaf)
            row[N.FT_LEAF0 + 3 * li + 2] = slot_base[leaf]
        return row

    def _leaf_transposed(self, i: int, sites: list[LoraSite]) -> bool:
        # pe rows are [r][M]; A leaves [d_in, r] need the transpose, B leaves [r, d_out] do not.
        for s in sites:
            if s.a_leaf == i:
                return not s.a_transposed
            if s.b_leaf == i:
                return s.b_transposed
        return False

    def linear_finite(self) -> torch.Tensor:
        """Device bool: no per-example weight gradient of a linear site held a
        non-finite entry in the last run (outer-form norms flag them; the
        other sites' column masks record them)."""
        ok = self._part_buf[-1:].view(torch.int64)[0] == 0
        if self._has_masks:
            ok = ok & (self.nf_mask == 0).all()
        return ok

    def rank_planes(self, site: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The rank-space products of LoRA site ``site`` (its index in the
        plan's site list) as the last run laid them out: V = x A and
        U = g B^T, [n_rows, r] views of the plan's planes.  Rows outside the
        segments are 0 or unspecified."""
        dt, vbase, ubase, c0, r, ldq, n_rows = self._planes_of[site]
        q = self.qbuf[dt]

        def view(base: int) -> torch.Tensor:
            return q[base + c0 * ldq : base + (c0 + r) * ldq].view(r, ldq)[:, :n_rows].t()

        return view(vbase), view(ubase)

    def pe_views(self) -> list[torch.Tensor]:
        """The per-example factor gradients each LoRA leaf stored ([n_seg * r * M], parameter dtype)."""
        return [self.pe[dt][o : o + n] for dt, o, n in self._pe_slices]

    # -- execution -------------------------------------------------------------
    def run(self, events: dict | None = None, launch_log: list | None = None) -> GhostResult:
        """Launch the step on the current stream.

        ``events`` may map a stage name ("project", "factor_project",
        "factor", "sqnorm", "nonfinite", "lin_norm", "clip", "scale_sum", "lin_sum") to a
        (start, end) pair of torch.cuda.Event that are recorded around that
        stage's launches ("lin_sum" spans the clipped sums of full weights:
        their prescale, GEMM and moments launches).  ``launch_log``, when a
        list, receives one (stage, key, start, end) entry per table launch
        with freshly recorded timing events, in ``launch_info`` order.
        """
        lib = N.load()
        main = torch.cuda.current_stream()
        stream = main.cuda_stream
        seg = self.segments
        ev = events or {}
        self._part_buf.zero_()
        if self._amax.numel():
            self._amax.zero_()
        live = [t for t in self.tables if t[5] > 0 and t[0] not in _AFTER_CLIP]

        def mark(name, dt, on):
            if launch_log is None:
                return None
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(on)
            launch_log.append((name, dt, e0, e1))
            return e1

        def launch(name, dt, probs, ws, n, total, s):
            if name == "pack":
                N.check(lib.odp_pack_factors(s, probs.data_ptr(), ws.data_ptr(), n, total), name)
            elif name == "planes":
                N.check(lib.odp_pack_planes(s, probs.data_ptr(), ws.data_ptr(), n, total,
                                            self.seg_start.data_ptr(), self.seg_len.data_ptr()), name)
            elif name == "project":
                N.check(lib.odp_project(s, dtype_code(dt[0]), probs.data_ptr(), ws.data_ptr(), n, total,
                                        self.seg_start.data_ptr(), self.seg_len.data_ptr(), dt[1]), name)
            elif name == "factor_project":
                N.check(lib.odp_seg_factor_project(s, probs.data_ptr(), ws.data_ptr(), n, total,
                                                   self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                                   self.seg_ex.data_ptr(), self.part.data_ptr(),
                                                   self.n_slots), name)
            elif name == "factor_stream":
                N.check(lib.odp_seg_factor_stream(s, probs.data_ptr(), ws.data_ptr(), n, total,
                                                  self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                                  self.seg_ex.data_ptr(), self.part.data_ptr(),
                                                  self.n_slots, dt), name)
            elif name == "factor":
                N.check(lib.odp_seg_factor(s, dtype_code(dt[0]), probs.data_ptr(), ws.data_ptr(), n, total,
                                           self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                           self.seg_ex.data_ptr(), self.part.data_ptr(), self.n_slots,
                                           dt[1]), name)
            elif name == "sqnorm":
                N.check(lib.odp_sqnorm(s, probs.data_ptr(), ws.data_ptr(), n, total,
                                       self.seg_ex.data_ptr(), self.part.data_ptr(), self.n_slots), name)
            elif name == "nonfinite":
                N.check(lib.odp_nonfinite_columns(s, probs.data_ptr(), ws.data_ptr(), n, total,
                                                  self.seg_start.data_ptr(), self.seg_len.data_ptr()), name)
            elif name == "lin_norm":
                N.check(lib.odp_linear_sqnorm(s, dt, probs.data_ptr(), ws.data_ptr(), n, total,
                                              self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                              self.seg_ex.data_ptr(), self.part.data_ptr(), self.n_slots), name)

        # Every table on the caller's stream, in table order.  (Launching the
        # tables of one stage side by side on forked streams, to overlap each
        # launch's last round of workgroups with the next, measured no faster
        # on MI355X.)
        names = [t[0] for t in live]
        for idx, (name, dt, probs, ws, n, total) in enumerate(live):
            if name in ev and name not in names[:idx]:
                ev[name][0].record(main)
            end_ev = mark(name, dt, main)
            launch(name, dt, probs, ws, n, total, stream)
            if end_ev is not None:
                end_ev.record(main)
            if name in ev and name not in names[idx + 1:]:
                ev[name][1].record(main)
        if "clip" in ev:
            ev["clip"][0].record()
        N.check(
            lib.odp_clip_factors(
                stream, self.part.data_ptr(), self.n_slots, seg.n_ex, self.gstart.data_ptr(), self.n_groups,
                self.thr.data_ptr(), float(self.clip.effective), int(self.clip.mode), float(self.clip.gamma),
                self.n_cls, self.guard.data_ptr(), self.cls_dt.data_ptr(), self.scales.data_ptr(),
                self.norms.data_ptr(), self.group_norms.data_ptr(), self.clipped.data_ptr(),
                self.clipped_total.data_ptr(),
            ),
            "odp_clip_factors",
        )
        if "clip" in ev:
            ev["clip"][1].record()
        post = [t for t in self.tables if t[5] > 0 and t[0] in _AFTER_CLIP]
        stage = [("lin_sum" if t[0] in ("lin_prescale", "lin_moments") else t[0]) for t in post]
        for idx, (name, dt, probs, ws, n, total) in enumerate(post):
            st = stage[idx]
            if st in ev and st not in stage[:idx]:
                ev[st][0].record()
            end_ev = mark(name, dt, main)
            if name == "scale_sum":
                N.check(lib.odp_scale_sum(stream, probs.data_ptr(), ws.data_ptr(), n, total,
                                          self.seg_ex.data_ptr(), self.scales.data_ptr(), seg.n_ex,
                                          self.n_groups, float(self.clip.normalize_by)), name)
            elif name == "lin_prescale":
                N.check(lib.odp_linear_prescale(stream, probs.data_ptr(), ws.data_ptr(), n, total,
                                                self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                                self.seg_ex.data_ptr(), self.scales.data_ptr(), seg.n_ex,
                                                self.n_groups), name)
            elif name == "lin_sum":
                N.check(lib.odp_linear_clipped_sum(stream, probs.data_ptr(), ws.data_ptr(), n, total,
                                                   self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                                   self.seg_ex.data_ptr(), self.scales.data_ptr(), seg.n_ex,
                                                   self.n_groups, float(self.clip.normalize_by),
                                                   0 if dt is None else 1), name)
            elif name == "lin_moments":
                N.check(lib.odp_linear_moments(stream, probs.data_ptr(), ws.data_ptr(), n, total,
                                               self.seg_start.data_ptr(), self.seg_len.data_ptr(),
                                               self.seg_ex.data_ptr(), self.scales.data_ptr(), seg.n_ex,
                                               self.n_groups, float(self.clip.normalize_by),
                                               0 if dt is None else 1), name)
            if end_ev is not None:
                end_ev.record()
            if st in ev and st not in stage[idx + 1:]:
                ev[st][1].record()
        return GhostResult(
            leaves=self.out,
            norms=self.norms,
            group_norms=self.group_norms,
            clipped=self.clipped,
            clipped_total=self.clipped_total,
            scales=self.scales,
            second_moment=self.out2,
            flat=self.flat,
        )


__all__ = [
    "plan_key",
    "ClipSpec",
    "GhostPlan",
    "GhostResult",
    "LeafOut",
    "LoraSite",
    "MaterializedLeaf",
    "Segments",
    "dtype_code",
    "supports_rows",
]
