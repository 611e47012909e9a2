"""Host side of the MI355X sampling step: ctypes binding of libarbor_hip.so and the
``Sampling`` op that mirrors the managed API a caller of ArborNet would use.

The reference binds its native kernels through P/Invoke declarations
(ArborNet.Core/Native/PInvoke/CUDA.cs:90-202) and surfaces ops as static methods
(ArborNet.Core/Functional/Ops.cs:21-393, e.g. ``Ops.Softmax`` at :327). A nonzero native
status becomes an exception carrying the native message, as ``CUDA.Check`` turns a
CudaError into InvalidOperationException (CUDA.cs:360-364). This module does the same in
Python: ``Sampling.sample`` validates nothing itself (the library does), launches on the
current torch stream, and raises :class:`ArborSamplingError` on any nonzero status.

torch is used only for device buffers and the stream handle; all computation happens in
the HIP library. There is no CPU fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path
from typing import Optional

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libarbor_hip.so"
HEADER_PATH = _PKG.parent / "include" / "arbor_sampling.h"

ARBOR_DTYPE_F32 = 0
ARBOR_DTYPE_BF16 = 1
ARBOR_FLAG_WRITE_PROBS = 1

ARBOR_ID_EMPTY = -1
ARBOR_ID_INVALID = -2
ARBOR_ID_BAD_HISTORY = -3
ARBOR_ID_STALLED = -4
ARBOR_VOCAB_MAX = 1048575

STATUS_NAMES = {
    0: "ARBOR_OK",
    -1: "ARBOR_ERR_NULL",
    -2: "ARBOR_ERR_STRUCT_SIZE",
    -3: "ARBOR_ERR_SHAPE",
    -4: "ARBOR_ERR_DTYPE",
    -5: "ARBOR_ERR_TEMPERATURE",
    -6: "ARBOR_ERR_PENALTY",
    -7: "ARBOR_ERR_TOP_K",
    -8: "ARBOR_ERR_TOP_P",
    -9: "ARBOR_ERR_MIN_P",
    -10: "ARBOR_ERR_HISTORY",
    -11: "ARBOR_ERR_MASK",
    -12: "ARBOR_ERR_WORKSPACE",
    -13: "ARBOR_ERR_FLAGS",
    -14: "ARBOR_ERR_NO_DEVICE",
}


class ArborSamplingError(RuntimeError):
    """A nonzero status from libarbor_hip (negative: argument error, positive: HIP error)."""

    def __init__(self, status: int, message: str):
        self.status = status
        name = STATUS_NAMES.get(status, f"hipError {status}")
        super().__init__(f"{name}: {message}")


class SamplingParams(ctypes.Structure):
    """Mirror of ``arbor_sampling_params`` (include/arbor_sampling.h)."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("batch", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("ld_logits", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("temperature", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("hist_len", ctypes.c_int32),
        ("mask_words", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]

    # integer fields whose C type is int32_t: ctypes would wrap larger values silently
    _INT32_FIELDS = ("batch", "vocab", "ld_logits", "dtype", "top_k", "hist_len", "mask_words")

    @classmethod
    def make(cls, batch: int, vocab: int, **kw) -> "SamplingParams":
        """Params with the library's defaults, overridden by ``kw``. Integer fields must fit
        int32: a row stride of 2^31 elements or more (e.g. ``ld_logits = seq * vocab`` of a
        long [batch, seq, vocab] output) raises ARBOR_ERR_SHAPE instead of wrapping."""
        vals = dict(batch=batch, vocab=vocab, ld_logits=vocab, dtype=ARBOR_DTYPE_F32, temperature=1.0,
                    repetition_penalty=1.0, top_p=1.0, mask_words=(vocab + 31) // 32)
        vals.update(kw)
        p = cls()
        p.struct_size = ctypes.sizeof(cls)
        for k, v in vals.items():
            if not hasattr(p, k):
                raise AttributeError(k)
            if k in cls._INT32_FIELDS and not (-2**31 <= int(v) < 2**31):
                raise ArborSamplingError(-3, f"{k} = {int(v)} does not fit int32 (the ABI field is int32_t)")
            setattr(p, k, v)
        return p

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_lib = None


def library() -> ctypes.CDLL:
    """Load libarbor_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m arbornet_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        P = ctypes.POINTER(SamplingParams)
        lib.arbor_sample.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.arbor_sample.restype = i32
        lib.arbor_sample_append.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.arbor_sample_append.restype = i32
        lib.arbor_decode.argtypes = [vp, ctypes.c_int32, vp, vp, ctypes.c_int32, ctypes.c_int32, vp, vp, sz, vp]
        lib.arbor_decode.restype = i32
        lib.arbor_embed.argtypes = [vp, ctypes.c_int32, vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, vp, vp]
        lib.arbor_embed.restype = i32
        lib.arbor_lm_head_packed_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32]
        lib.arbor_lm_head_packed_bytes.restype = sz
        lib.arbor_lm_head_pack.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, vp, vp]
        lib.arbor_lm_head_pack.restype = i32
        lib.arbor_lm_head.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, vp, vp, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_float, vp, ctypes.c_int32, ctypes.c_int32, vp, vp]
        lib.arbor_lm_head.restype = i32
        lib.arbor_sample_noalloc.argtypes = [P, vp, vp, vp, vp, vp, vp, vp]
        lib.arbor_sample_noalloc.restype = i32
        lib.arbor_sample_workspace_bytes.argtypes = [P]
        lib.arbor_sample_workspace_bytes.restype = sz
        lib.arbor_sampling_params_init.argtypes = [P, ctypes.c_int32, ctypes.c_int32]
        lib.arbor_sampling_params_init.restype = None
        lib.arbor_device_count.argtypes = [ctypes.POINTER(ctypes.c_int)]
        lib.arbor_device_count.restype = i32
        lib.arbor_malloc.argtypes = [ctypes.POINTER(vp), sz]
        lib.arbor_malloc.restype = i32
        lib.arbor_free.argtypes = [vp]
        lib.arbor_free.restype = i32
        lib.arbor_memcpy.argtypes = [vp, vp, sz, i32]
        lib.arbor_memcpy.restype = i32
        lib.arbor_memset.argtypes = [vp, i32, sz]
        lib.arbor_memset.restype = i32
        lib.arbor_synchronize.argtypes = []
        lib.arbor_synchronize.restype = i32
        lib.arbor_last_error.argtypes = []
        lib.arbor_last_error.restype = ctypes.c_char_p
        lib.arbor_abi_version.argtypes = []
        lib.arbor_abi_version.restype = i32
        _lib = lib
    return _lib


def header_functions() -> list[str]:
    """Names of the functions include/arbor_sampling.h declares."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(arbor_[a-z_0-9]+)\s*\(", text, flags=re.M)


def check(status: int) -> None:
    if status != 0:
        msg = library().arbor_last_error().decode(errors="replace")
        raise ArborSamplingError(status, msg)


def workspace_bytes(params: SamplingParams) -> int:
    return int(library().arbor_sample_workspace_bytes(ctypes.byref(params)))


def sample_raw(params: SamplingParams, logits: int, history: Optional[int], mask: Optional[int],
               uniforms: int, out_ids: int, out_probs: Optional[int], workspace: int,
               workspace_bytes_: int, stream: Optional[int]) -> int:
    """Call arbor_sample with raw device addresses; returns the status (does not raise)."""
    return int(library().arbor_sample(ctypes.byref(params), logits, history, mask, uniforms, out_ids,
                                      out_probs, workspace, workspace_bytes_, stream))


def sample_noalloc_raw(params: SamplingParams, logits: int, history: Optional[int], mask: Optional[int],
                       uniforms: int, out_ids: int, out_probs: Optional[int], stream: Optional[int]) -> int:
    """Call arbor_sample_noalloc (the library's static scratch is the workspace); returns
    the status."""
    return int(library().arbor_sample_noalloc(ctypes.byref(params), logits, history, mask, uniforms, out_ids,
                                              out_probs, stream))


def sample_append_raw(params: SamplingParams, logits: int, history: int, positions: int, mask: Optional[int],
                      uniforms: int, out_ids: int, out_probs: Optional[int], workspace: int,
                      workspace_bytes_: int, stream: Optional[int]) -> int:
    """Call arbor_sample_append with raw device addresses; returns the status."""
    return int(library().arbor_sample_append(ctypes.byref(params), logits, history, positions, mask, uniforms,
                                             out_ids, out_probs, workspace, workspace_bytes_, stream))


_workspaces: dict = {}


def _workspace(device, stream: int, nbytes: int):
    """A workspace of at least nbytes on `device` for calls launched on `stream` (a raw
    stream handle), cached per (device, stream). Calls that share a workspace must be
    ordered, and calls on one stream are; calls on different streams get different
    buffers. A buffer is allocated while its stream is torch's current stream, so the
    caching allocator hands its memory, once replaced and freed, only to later work on
    that same stream."""
    import torch

    key = (device.type, device.index, int(stream or 0))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        _workspaces.pop(key, None)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


class Sampling:
    """The sampling op, as the managed ``Sampling`` static class would expose it."""

    @staticmethod
    def sample(logits, uniforms, *, temperature: float = 1.0, repetition_penalty: float = 1.0,
               frequency_penalty: float = 0.0, presence_penalty: float = 0.0, top_k: int = 0,
               top_p: float = 1.0, min_p: float = 0.0, history=None, allow_mask=None,
               vocab: Optional[int] = None, write_probs: bool = False, out_ids=None, out_probs=None):
        """Sample one token id per row of ``logits`` ([batch, ld] fp32 or bf16 on a HIP
        device). ``vocab`` defaults to the row length; ``history`` is [batch, H] int32
        (-1 = padding), ``allow_mask`` [batch, >= ceil(vocab/32)] int32/uint32 bit words,
        ``uniforms`` [batch] fp32. Returns int32 ids [batch], or (ids, probs) if
        ``write_probs``."""
        import torch

        if logits.dim() != 2:
            raise ValueError("logits must be [batch, ld]")
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        dev = logits.device
        if dev.type != "cuda":
            raise ArborSamplingError(-14, "logits must live on a HIP device")
        batch = logits.shape[0]
        V = int(vocab) if vocab is not None else logits.shape[1]
        dtype = {torch.float32: ARBOR_DTYPE_F32, torch.bfloat16: ARBOR_DTYPE_BF16}.get(logits.dtype)
        if dtype is None:
            raise ArborSamplingError(-4, f"logits dtype {logits.dtype} is not float32 or bfloat16")
        p = SamplingParams.make(batch, V, ld_logits=logits.stride(0), dtype=dtype, temperature=temperature,
                                repetition_penalty=repetition_penalty, frequency_penalty=frequency_penalty,
                                presence_penalty=presence_penalty, top_k=top_k, top_p=top_p, min_p=min_p)
        hist_ptr = mask_ptr = None
        if history is not None:
            history = history.to(device=dev, dtype=torch.int32).contiguous()
            p.hist_len = history.shape[1]
            hist_ptr = history.data_ptr()
        if allow_mask is not None:
            if allow_mask.dtype not in (torch.int32, torch.uint32):
                raise ValueError("allow_mask must be int32/uint32 bit words")
            allow_mask = allow_mask.to(device=dev).contiguous()
            p.mask_words = allow_mask.shape[1]
            mask_ptr = allow_mask.data_ptr()
        uniforms = uniforms.to(device=dev, dtype=torch.float32).contiguous()
        if uniforms.numel() != batch:
            raise ValueError("one uniform per row is required")
        if out_ids is None:
            out_ids = torch.empty(batch, dtype=torch.int32, device=dev)
        probs_ptr = None
        if write_probs:
            p.flags |= ARBOR_FLAG_WRITE_PROBS
            if out_probs is None:
                out_probs = torch.empty((batch, V), dtype=torch.float32, device=dev)
            probs_ptr = out_probs.data_ptr()
        need = workspace_bytes(p)
        if need == 0:  # invalid params: let arbor_sample report why
            need = 256
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = _workspace(dev, stream, need)
        check(sample_raw(p, logits.data_ptr(), hist_ptr, mask_ptr, uniforms.data_ptr(), out_ids.data_ptr(),
                         probs_ptr, ws.data_ptr(), ws.numel(), stream))
        return (out_ids, out_probs) if write_probs else out_ids


def params_for(workload, write_probs: bool = False) -> SamplingParams:
    """SamplingParams of a synthetic.Workload."""
    return SamplingParams.make(
        workload.batch, workload.vocab, ld_logits=workload.row_stride,
        dtype=ARBOR_DTYPE_BF16 if workload.dtype == "bf16" else ARBOR_DTYPE_F32,
        temperature=workload.temperature, repetition_penalty=workload.repetition_penalty,
        frequency_penalty=workload.frequency_penalty, presence_penalty=workload.presence_penalty,
        top_k=workload.top_k, top_p=workload.top_p, min_p=workload.min_p, hist_len=workload.hist_len,
        mask_words=workload.mask_words, flags=ARBOR_FLAG_WRITE_PROBS if write_probs else 0)


class GenerationState:
    """Per-row token history of a generation loop, resident on the device: a ring of
    ``hist_len`` ids per row (-1 = empty) and the number of ids appended to each row.
    ``step`` samples from the last position of the model's logits and appends the sampled
    ids (arbor_sample_append), so that the next step's penalties count them. There is no
    counterpart in the reference: its models' Forward (ArborNet.Models/GPT.cs:96-111,
    Llama3.cs:67-74) returns [batch, seq, vocab] logits that nothing consumes."""

    def __init__(self, batch: int, hist_len: int, device, prompt=None):
        import torch

        if hist_len <= 0:
            raise ValueError("hist_len must be positive")
        self.batch, self.hist_len, self.device = batch, hist_len, torch.device(device)
        self.history = torch.full((batch, hist_len), -1, dtype=torch.int32, device=self.device)
        self.positions = torch.zeros(batch, dtype=torch.int32, device=self.device)
        if prompt is not None:  # [batch, P] prompt ids: the last hist_len of them seed the ring
            prompt = torch.as_tensor(prompt, dtype=torch.int32)
            tail = prompt[:, -hist_len:]
            self.history[:, : tail.shape[1]] = tail.to(self.device)
            self.positions.fill_(tail.shape[1] % hist_len)

    def step(self, logits, uniforms, *, temperature: float = 1.0, repetition_penalty: float = 1.0,
             frequency_penalty: float = 0.0, presence_penalty: float = 0.0, top_k: int = 0,
             top_p: float = 1.0, min_p: float = 0.0, allow_mask=None, vocab: Optional[int] = None,
             out_ids=None):
        """Sample one id per row from ``logits`` ([batch, seq, vocab]: the last position is
        used; or [batch, ld]) and append it to the history. Returns int32 ids [batch]."""
        import torch

        if logits.dim() == 3:
            logits = logits[:, -1, :]
        if logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be [batch, seq, vocab] or [batch, ld] with contiguous rows")
        if logits.shape[0] != self.batch or logits.device != self.device:
            raise ValueError("logits do not match this state's batch and device")
        V = int(vocab) if vocab is not None else logits.shape[1]
        dtype = {torch.float32: ARBOR_DTYPE_F32, torch.bfloat16: ARBOR_DTYPE_BF16}.get(logits.dtype)
        if dtype is None:
            raise ArborSamplingError(-4, f"logits dtype {logits.dtype} is not float32 or bfloat16")
        p = SamplingParams.make(self.batch, V, ld_logits=logits.stride(0), dtype=dtype, temperature=temperature,
                                repetition_penalty=repetition_penalty, frequency_penalty=frequency_penalty,
                                presence_penalty=presence_penalty, top_k=top_k, top_p=top_p, min_p=min_p,
                                hist_len=self.hist_len)
        mask_ptr = None
        if allow_mask is not None:
            allow_mask = allow_mask.to(device=self.device).contiguous()
            p.mask_words = allow_mask.shape[1]
            mask_ptr = allow_mask.data_ptr()
        uniforms = uniforms.to(device=self.device, dtype=torch.float32).contiguous()
        if out_ids is None:
            out_ids = torch.empty(self.batch, dtype=torch.int32, device=self.device)
        need = workspace_bytes(p) or 256
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ws = _workspace(self.device, stream, need)
        check(sample_append_raw(p, logits.data_ptr(), self.history.data_ptr(), self.positions.data_ptr(), mask_ptr,
                                uniforms.data_ptr(), out_ids.data_ptr(), None, ws.data_ptr(), ws.numel(), stream))
        return out_ids


class TokenTable:
    """A tokenizer vocabulary on the device as an id -> bytes table (CSR), for decoding
    sampled ids in one launch (arbor_decode). Mirrors the reference's Decode
    (ArborNet.Data/Tokenizers.cs:191-200, :304-313): the text of id t is the first key of the
    vocabulary (in its order) that maps to t, the unknown token when none does or t lies
    outside the vocabulary; the texts are joined with nothing between them."""

    def __init__(self, vocab: dict, unk_token: str, device="cuda"):
        import numpy as np
        import torch

        n = max(vocab.values(), default=-1) + 1
        text = [None] * n
        for key, v in vocab.items():
            if 0 <= v < n and text[v] is None:
                text[v] = key
        self.vocab = n
        self.unk_id = vocab.get(unk_token, -1)
        blobs = [(t if t is not None else unk_token).encode("utf-8") for t in text]
        offsets = np.zeros(n + 1, dtype=np.int32)
        offsets[1:] = np.cumsum([len(b) for b in blobs], dtype=np.int64)
        data = np.frombuffer(b"".join(blobs) or b"\0", dtype=np.uint8).copy()
        self.offsets = torch.from_numpy(offsets).to(device)
        self.bytes = torch.from_numpy(data).to(device)
        self.device = torch.device(device)

    def decode_raw(self, ids, capacity: Optional[int] = None):
        """(out_offsets [count + 1], out_bytes) of device ids (int32 tensor), on the current
        stream; raises ArborSamplingError on a nonzero status."""
        import torch

        ids = ids.to(device=self.device, dtype=torch.int32).contiguous()
        count = ids.numel()
        cap = 64 * max(count, 1) if capacity is None else capacity
        offs = torch.empty(count + 1, dtype=torch.int32, device=self.device)
        out = torch.empty(max(cap, 1), dtype=torch.uint8, device=self.device)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        check(int(library().arbor_decode(ids.data_ptr(), count, self.offsets.data_ptr(), self.bytes.data_ptr(),
                                         self.vocab, self.unk_id, offs.data_ptr(), out.data_ptr(), cap, stream)))
        return offs, out

    def decode(self, ids) -> str:
        """The text of a batch of ids (one launch; a second one if the first ran out of room)."""
        offs, out = self.decode_raw(ids)
        total = int(offs[-1].item())
        if total > out.numel():
            offs, out = self.decode_raw(ids, capacity=total)
        return bytes(out[:total].cpu().numpy()).decode("utf-8", errors="replace")


def embed(ids, table, out=None):
    """out[i, :] = table[ids[i], :] on the device (zeros for ids outside the table), the
    embedding gather a generation loop feeds its next forward pass (arbor_embed)."""
    import torch

    if table.dim() != 2 or not table.is_contiguous():
        raise ValueError("table must be a contiguous [vocab, width] tensor")
    dtype = {torch.float32: ARBOR_DTYPE_F32, torch.bfloat16: ARBOR_DTYPE_BF16}.get(table.dtype)
    if dtype is None:
        raise ArborSamplingError(-4, f"table dtype {table.dtype} is not float32 or bfloat16")
    ids = ids.to(device=table.device, dtype=torch.int32).contiguous()
    if out is None:
        out = torch.empty((ids.numel(), table.shape[1]), dtype=table.dtype, device=table.device)
    stream = torch.cuda.current_stream(table.device).cuda_stream
    check(int(library().arbor_embed(ids.data_ptr(), ids.numel(), table.data_ptr(), table.shape[0], table.shape[1],
                                    dtype, out.data_ptr(), stream)))
    return out


ARBOR_LM_WEIGHT_HV = 0  # weight [hidden, vocab]: the reference's Linear.weight (in x out)
ARBOR_LM_WEIGHT_VH = 1  # weight [vocab, hidden]


def _dtype_code(t):
    import torch

    code = {torch.float32: ARBOR_DTYPE_F32, torch.bfloat16: ARBOR_DTYPE_BF16}.get(t.dtype)
    if code is None:
        raise ArborSamplingError(-4, f"dtype {t.dtype} is not float32 or bfloat16")
    return code


class LMHead:
    """The logits producer before the sampler, on the matrix cores: logits = (x @ W + bias)
    * scale with bf16 operands and fp32 accumulation (arbor_lm_head). Mirrors the reference's
    Linear.Forward, input.MatMul(weight).Add(bias) (ArborNet.Layers/Linear.cs:29), whose weight
    is [in, out] = [hidden, vocab] (layout "hv"); "vh" takes a [vocab, hidden] weight. The
    weight is packed once, here, into the order the matrix instructions read."""

    def __init__(self, weight, bias=None, layout: str = "hv"):
        import torch

        if weight.dim() != 2 or not weight.is_contiguous():
            raise ValueError("weight must be a contiguous 2-D tensor")
        lay = {"hv": ARBOR_LM_WEIGHT_HV, "vh": ARBOR_LM_WEIGHT_VH}[layout]
        self.hidden, self.vocab = (weight.shape[0], weight.shape[1]) if lay == ARBOR_LM_WEIGHT_HV else \
            (weight.shape[1], weight.shape[0])
        self.device = weight.device
        nbytes = int(library().arbor_lm_head_packed_bytes(self.hidden, self.vocab))
        if nbytes == 0:
            raise ArborSamplingError(-3, f"hidden {self.hidden} must be a positive multiple of 128, vocab {self.vocab} "
                                         f"in (0, {ARBOR_VOCAB_MAX}]")
        self.packed = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        check(int(library().arbor_lm_head_pack(weight.data_ptr(), _dtype_code(weight), lay, self.hidden, self.vocab,
                                               self.packed.data_ptr(), stream)))
        self.bias = None if bias is None else bias.to(device=self.device, dtype=torch.float32).contiguous()

    def __call__(self, x, scale: float = 1.0, out_dtype=None, out=None, row_max: bool = False):
        """x [batch, hidden] (rows may be strided) -> logits [batch, vocab] (fp32 unless
        out_dtype or out says bf16), and the rows' maxima if row_max."""
        import torch

        if x.dim() != 2 or x.shape[1] != self.hidden or x.stride(1) != 1:
            raise ValueError(f"x must be [batch, {self.hidden}] with unit column stride")
        B = x.shape[0]
        if out is None:
            out = torch.empty((B, self.vocab), dtype=out_dtype or torch.float32, device=self.device)
        if out.dim() != 2 or out.shape[0] != B or out.shape[1] < self.vocab or out.stride(1) != 1:
            raise ValueError("out must be [batch, >= vocab] with unit column stride")
        rm = torch.empty(B, dtype=torch.float32, device=self.device) if row_max else None
        stream = torch.cuda.current_stream(self.device).cuda_stream
        check(int(library().arbor_lm_head(
            x.data_ptr(), _dtype_code(x), B, x.stride(0), self.packed.data_ptr(),
            None if self.bias is None else self.bias.data_ptr(), self.hidden, self.vocab, float(scale),
            out.data_ptr(), _dtype_code(out), out.stride(0), None if rm is None else rm.data_ptr(), stream)))
        return (out, rm) if row_max else out
