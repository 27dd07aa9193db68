"""Dispatch layer: drop-in for the reference's src/ops.py.

One implementation serves every entry point: the HIP kernels of libfdi4 on
the GPU, reached through the torch binding ``_C``. The names, signatures,
return types and error behaviour of the reference are kept
(src/ops.py:86-344): ``quantize_int4``, ``flash_decode``,
``prepare_quantize_int4_cuda``, ``prepare_flash_decode_cuda``,
``backend_status``, ``QUANTIZE_BACKENDS``, ``ATTENTION_BACKENDS``,
``CUDA_MAX_HEAD_DIM``, ``HAS_CUDA``.

Backends. ``"hip"`` is the implementation; ``"cuda"`` is accepted as its
alias because PyTorch-ROCm names the GPU device ``cuda``. There is no CPU
path: ``backend="reference"`` (the NumPy oracle, which this package does not
ship), ``use_cuda=False``, ``"triton"`` and ``"pallas"`` raise, and every op
raises ``RuntimeError`` when the extension or the GPU is missing. A named
backend is delivered or refused, never substituted (reference
src/ops.py:90-108).

Beyond the reference: ``quantize_int4_paged`` / ``flash_decode_paged`` (the
per-sequence paged layout with 128-token scale groups and packed keys) and
``pack_int4_device``.
"""

from typing import List, Optional, Tuple

import numpy as np

from ._lib import binding_available, gpu_available, load_binding
from ._prepared import PreparedCall
from ._validate import normalize_attention_inputs

try:
    import torch
    HAS_TORCH = True
except ImportError:  # pragma: no cover
    torch = None
    HAS_TORCH = False

HAS_EXTENSION = binding_available()
#: True when the HIP extension is built and a GPU is visible.
HAS_HIP = HAS_EXTENSION and gpu_available()
HAS_CUDA = HAS_HIP


def __getattr__(name):
    # ``ops._C`` is the torch binding, loaded on first use (so that a build in
    # the same process after this module was imported is picked up).
    if name == "_C":
        return load_binding()
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


QUANTIZE_BACKENDS = ("hip", "cuda")
ATTENTION_BACKENDS = ("hip", "cuda")

#: Widest head the attention path accepts (heads are padded to 64/128/256
#: channels on the device). reference: src/ops.py:164-166.
HIP_MAX_HEAD_DIM = 256
CUDA_MAX_HEAD_DIM = HIP_MAX_HEAD_DIM

_PAD_DIMS = (64, 128, 256)


def _padded_dim(d: int) -> int:
    for p in _PAD_DIMS:
        if d <= p:
            return p
    raise ValueError(f"head_dim {d} exceeds {HIP_MAX_HEAD_DIM}")


def _validate_backend(backend: Optional[str], supported: tuple, op: str) -> None:
    """Reject unknown or unavailable backends instead of substituting one."""
    if backend is None or backend in supported:
        return
    if backend == "reference":
        raise ValueError(
            "backend 'reference' is the NumPy oracle, which is test infrastructure and not "
            f"part of this package; supported backends for {op}: {supported}")
    if backend in ("triton", "pallas"):
        raise ValueError(
            f"no {backend} kernels exist in this package (HIP only); supported backends for "
            f"{op}: {supported}")
    raise ValueError(f"unknown backend {backend!r} for {op}; supported: {supported}")


def _require_device(use_cuda: Optional[bool]) -> None:
    if use_cuda is False:
        raise RuntimeError(
            "use_cuda=False asks for a CPU implementation; this package has none (the kernels "
            "run on the GPU only)")
    if not HAS_EXTENSION:
        load_binding()  # raises with the reason
    if not gpu_available():
        raise RuntimeError("the HIP backend needs a visible GPU (torch.cuda.is_available() "
                           "is False)")


def _sync(_out=None) -> None:
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# quantizer
# ---------------------------------------------------------------------------

def prepare_quantize_int4_hip(kv) -> PreparedCall:
    """Stage a 2-D [rows, channels] array on the GPU once; run() enqueues the quantizer."""
    _require_device(None)
    if isinstance(kv, torch.Tensor):
        kv_t = kv.to(device="cuda", dtype=torch.float32).contiguous()
    else:
        kv_t = torch.from_numpy(np.ascontiguousarray(kv, dtype=np.float32)).cuda()
    if kv_t.dim() != 2:
        raise ValueError(f"the HIP quantizer takes a 2D [rows, channels] array, got shape "
                         f"{tuple(kv_t.shape)}")
    C = load_binding()
    return PreparedCall(
        run=lambda: C.quantize_int4(kv_t),
        sync=_sync,
        to_numpy=lambda out: tuple(t.cpu().numpy() for t in out),
    )


prepare_quantize_int4_cuda = prepare_quantize_int4_hip


def quantize_int4(kv, use_cuda: Optional[bool] = None, backend: Optional[str] = None,
                  interpret: Optional[bool] = None):
    """Per-channel asymmetric INT4 quantization: one scale group over every row.

    Args:
        kv: [rows, channels] float32/float16 array (NumPy, or a torch tensor,
            in which case torch tensors on the GPU are returned). With
            ``backend=None`` higher-rank input is accepted and reduced over
            all leading axes, as the reference quantizer does.
        use_cuda: legacy flag; False raises (no CPU path).
        backend: "hip" / "cuda" or None.
        interpret: accepted for signature compatibility (Pallas-only in the reference).

    Returns:
        (q uint8 one value per byte, scale [channels], zp [channels]); bins
        bit-exact with the reference's NumPy quantizer.
    """
    _validate_backend(backend, QUANTIZE_BACKENDS, "quantize")
    _require_device(use_cuda)
    is_tensor = isinstance(kv, torch.Tensor)
    shape = tuple(kv.shape)
    if len(shape) != 2:
        if backend is not None:
            raise ValueError(
                f"the HIP quantizer takes a 2D [rows, channels] array, got shape {shape}. "
                "Use backend=None to reduce over all leading axes.")
        if len(shape) < 2:
            raise ValueError(f"KV must be at least 2D, got {len(shape)}D")
        kv = kv.reshape(-1, shape[-1])
    call = prepare_quantize_int4_hip(kv)
    if is_tensor:
        out = call.run()
        q, s, z = out
        return q.reshape(shape), s, z
    q, s, z = call()
    return q.reshape(shape), s, z


def pack_int4_device(q, out_cols: int = 0):
    """Device nibble packing of a [rows, channels] uint8 tensor (values taken mod 16)."""
    _require_device(None)
    return load_binding().pack_int4(q, out_cols)


def dequantize_int4(q, scale, zp, target_shape: Optional[Tuple] = None,
                    per_channel: bool = True, packed: bool = False,
                    num_channels: Optional[int] = None):
    """INT4 values back to float32 on the GPU: ``q*scale - zp*scale``, two
    rounded float32 products and a rounded subtraction, bit-exact with the
    reference's dequantize_int4_ref (src/quantize_int4_ref.py:87-136).

    Args:
        q: quantized values, one per byte (uint8, or any integer type with
           values in [0, 255]); with ``packed=True`` nibble pairs along the
           last axis (``pack_int4``), ``num_channels`` values per row
           (default: twice the bytes).
        scale, zp: per_channel -- the last axis's scales, broadcast over the
           leading axes (fewer dims are prepended, as in the reference);
           per-row -- the leading axes' scales, broadcast over the last axis
           (dims are appended). Any shape that then broadcasts to the output.
        target_shape: reshape the result to it.

    NumPy inputs give a NumPy result; torch tensors give a float32 tensor on
    the GPU.
    """
    _require_device(None)
    is_tensor = isinstance(q, torch.Tensor)
    dev = torch.device("cuda") if not is_tensor or not q.is_cuda else q.device
    qt = q if is_tensor else torch.from_numpy(np.ascontiguousarray(q))
    if qt.dim() < 1:
        raise ValueError("q must have at least one axis")
    if qt.dtype != torch.uint8:
        if qt.is_floating_point() or qt.is_complex() or qt.dtype == torch.bool:
            raise TypeError(f"q must hold integers, got {qt.dtype}")
        if qt.numel() and (int(qt.min()) < 0 or int(qt.max()) > 255):
            raise ValueError("q values must lie in [0, 255]")
        qt = qt.to(torch.uint8)
    qt = qt.to(dev)
    nbytes = qt.shape[-1]
    C = (num_channels if num_channels is not None else 2 * nbytes) if packed else nbytes
    if packed and nbytes != (C + 1) // 2:
        raise ValueError(f"{nbytes} packed bytes per row cannot hold {C} channels")
    out_shape = tuple(qt.shape[:-1]) + (C,)
    rows = int(np.prod(out_shape[:-1], dtype=np.int64))

    def _as_tensor(a):
        t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.asarray(a))
        t = t.to(device=dev, dtype=torch.float32)
        while t.dim() < len(out_shape):
            t = t.unsqueeze(0) if per_channel else t.unsqueeze(-1)
        try:
            return torch.broadcast_to(t, out_shape).reshape(rows, C)
        except RuntimeError as exc:
            raise ValueError(f"scale/zp of shape {tuple(a.shape)} do not broadcast to "
                             f"{out_shape}") from exc

    s2, z2 = _as_tensor(scale), _as_tensor(zp)
    if s2.stride() != z2.stride() or min(s2.stride()) < 0:
        s2, z2 = s2.contiguous(), z2.contiguous()
    q2 = qt.reshape(rows, nbytes)
    if q2.stride(1) != 1:
        q2 = q2.contiguous()
    out = load_binding().dequantize_int4(q2, s2, z2, int(C), bool(packed)).reshape(out_shape)
    if target_shape is not None:
        out = out.reshape(target_shape)
    if is_tensor:
        return out
    return out.cpu().numpy()


# ---------------------------------------------------------------------------
# attention over a list of pages (the reference's shared page stream)
# ---------------------------------------------------------------------------

def prepare_flash_decode_hip(query, k_q_blocks, k_scales, k_zps, v_blocks,
                             block_lens=None, num_splits: int = 0) -> PreparedCall:
    """Validate, pack, pad and stage inputs in HBM once; run() enqueues the decode.

    Pages are padded to the longest page's row count and head_dim to 64, 128
    or 256 channels; keys are nibble-packed; every (batch, head) query
    attends the same page stream (reference src/ops.py:189-192).
    """
    query, block_lens = normalize_attention_inputs(
        query, k_q_blocks, k_scales, k_zps, v_blocks, block_lens)
    nb = len(k_q_blocks)
    B, H, D = query.shape
    if nb == 0:
        zeros = np.zeros(query.shape, dtype=np.float32)
        return PreparedCall(run=lambda: zeros)
    if D > HIP_MAX_HEAD_DIM:
        raise ValueError(f"the HIP attention kernel supports head_dim <= {HIP_MAX_HEAD_DIM}, "
                         f"got {D}")
    _require_device(None)
    dp = _padded_dim(D)
    bs = max(int(np.shape(k)[0]) for k in k_q_blocks)
    bs = max(bs, 1)
    kq = np.zeros((nb, bs, dp), dtype=np.uint8)
    v = np.zeros((nb, bs, dp), dtype=np.float32)
    s = np.zeros((nb, dp), dtype=np.float32)
    z = np.zeros((nb, dp), dtype=np.float32)
    for i in range(nb):
        ki = np.asarray(k_q_blocks[i])
        n = ki.shape[0]
        if n and (ki.min() < 0 or ki.max() > 15):
            raise ValueError(f"key page {i} holds values outside [0, 15]")
        kq[i, :n, :D] = ki
        v[i, :n, :D] = v_blocks[i]
        s[i, :D] = k_scales[i]
        z[i, :D] = k_zps[i]
    packed = kq[..., 0::2] | (kq[..., 1::2] << 4)
    qp = np.zeros((B, H, dp), dtype=np.float32)
    qp[..., :D] = query
    dev = torch.device("cuda")
    q_t = torch.from_numpy(qp).to(dev)
    k_t = torch.from_numpy(np.ascontiguousarray(packed)).to(dev).view(nb, 1, bs, dp // 2)
    v_t = torch.from_numpy(v).to(dev).view(nb, 1, bs, dp)
    s_t = torch.from_numpy(s).to(dev)
    z_t = torch.from_numpy(z).to(dev)
    lens_t = torch.from_numpy(block_lens.astype(np.int32)).to(dev).view(1, nb).expand(B, nb)
    C = load_binding()

    def run():
        out = C.decode_paged(q_t, k_t, v_t, s_t, z_t, None, None, lens_t, 1, nb, num_splits)
        return out[..., :D]

    return PreparedCall(run=run, sync=_sync, to_numpy=lambda out: out.cpu().numpy())


prepare_flash_decode_cuda = prepare_flash_decode_hip


def flash_decode(query, k_q_blocks: List[np.ndarray], k_scales: List[np.ndarray],
                 k_zps: List[np.ndarray], v_blocks: List[np.ndarray],
                 block_lens: Optional[np.ndarray] = None, use_cuda: Optional[bool] = None,
                 backend: Optional[str] = None, interpret: Optional[bool] = None) -> np.ndarray:
    """Fused online-softmax attention over INT4 pages (reference src/ops.py:176-253).

    Every query in the [batch, heads] grid attends the same page stream.
    Logits are unscaled q.k; empty pages are skipped; zero pages give exact
    zeros. Returns float32 [batch, heads, head_dim].
    """
    _validate_backend(backend, ATTENTION_BACKENDS, "attention")
    query, block_lens = normalize_attention_inputs(
        query, k_q_blocks, k_scales, k_zps, v_blocks, block_lens)
    if len(k_q_blocks) == 0:
        # Attention over an empty cache: nothing accumulated, exact zeros.
        return np.zeros(query.shape, dtype=np.float32)
    if query.shape[2] > HIP_MAX_HEAD_DIM:
        raise ValueError(
            f"the HIP attention kernel supports head_dim <= {HIP_MAX_HEAD_DIM}, got "
            f"{query.shape[2]}")
    _require_device(use_cuda)
    return prepare_flash_decode_hip(query, k_q_blocks, k_scales, k_zps, v_blocks,
                                    block_lens)()


# ---------------------------------------------------------------------------
# paged layout: per-sequence page tables, group scales, packed keys
# ---------------------------------------------------------------------------

def quantize_int4_paged(k, seq_lens, page_table, k_pages, k_scale, k_zp,
                        group_rows: int = 128) -> None:
    """Quantize keys k[b, h, :seq_lens[b]] into packed pages and group scales.

    k float32 [B, Hkv, T, D] on the GPU (rows 16-byte aligned); seq_lens int32
    [B]; page_table int32 [B, max_pages]; k_pages uint8 [P, Hkv, page_rows,
    D/2]; k_scale, k_zp float32 [B, Hkv, ceil(T/group_rows), D]. Every
    group_rows tokens form one scale group (reference quantize_int4_ref applied
    per group, src/quantize_int4_ref.py:23-84); bit-exact.
    """
    _require_device(None)
    load_binding().quantize_paged(k, seq_lens, page_table, k_pages, k_scale, k_zp, group_rows)


def flash_decode_paged(query, k_pages, v_pages, k_scale, k_zp, page_table, seq_lens,
                       group_rows: int = 128, num_splits: int = 0, page_lens=None,
                       max_pages: Optional[int] = None):
    """Split-K fused INT4 flash decoding over the paged layout (all GPU tensors).

    query float32, float16 or bfloat16 [B, Hq, D]; k_pages uint8 [P, Hkv,
    page_rows, D/2]; v_pages float32, float16 or bfloat16 [P, Hkv, page_rows,
    D]; k_scale/k_zp [B, Hkv, G, D]; page_table int32 [B, max_pages] (or None
    for identity); seq_lens int32 [B] (or None with page_lens). q-head h reads
    kv-head h // (Hq // Hkv). Returns [B, Hq, D] on the GPU in the query's
    dtype: float32 arithmetic, 16-bit queries widened exactly, one rounding
    (to nearest even) of each output element.
    """
    _require_device(None)
    page_rows = k_pages.shape[2]
    if group_rows % page_rows:
        raise ValueError("group_rows must be a multiple of the page size")
    if max_pages is None:
        max_pages = page_table.shape[1] if page_table is not None else k_pages.shape[0]
    return load_binding().decode_paged(query, k_pages, v_pages, k_scale, k_zp, page_table,
                                       seq_lens, page_lens, group_rows // page_rows,
                                       int(max_pages), int(num_splits))


def backend_status() -> dict:
    """Availability of the (single) implementation. reference: src/ops.py:316-344."""
    status = {
        "has_torch": HAS_TORCH,
        "has_extension": HAS_EXTENSION,
        "has_hip": HAS_HIP,
        "has_cuda": HAS_CUDA,
        "gpu": gpu_available(),
        "active_backend": "hip" if HAS_HIP else "unavailable",
        "available_backends": ["hip", "cuda"] if HAS_HIP else [],
    }
    if HAS_EXTENSION:
        status["abi_version"] = int(load_binding().abi_version())
    if status["gpu"]:
        status["device"] = torch.cuda.get_device_name(0)
    return status
