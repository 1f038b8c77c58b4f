"""Python entry point of the MI355X fused FP8 MoE layer.

`run` has the signature, argument meaning, validation messages and destination-passing
behaviour of the reference's `run` (kernel.py:562-729). All arithmetic happens in the
gfx950 HIP library behind the C ABI of include/moe_fp8.h; this module only validates,
places tensors on the GPU, manages the per-stream workspace and passes raw pointers.
"""
from __future__ import annotations

import threading

import torch

from . import _lib
from ._lib import (BIAS_BF16, BIAS_F16, BIAS_F32, EXPERTS_GLOBAL, EXPERTS_LOCAL, G1_BLOCKS,
                   H_BLOCKS, HIDDEN, HIDDEN_BF16, HIDDEN_F16, HIDDEN_F32, I_BLOCKS, INTER, OUT_BF16,
                   OUT_F32, PACKED_MAX_TOKENS)

_BIAS_CODES = {torch.float32: BIAS_F32, torch.bfloat16: BIAS_BF16, torch.float16: BIAS_F16}


def _check_cuda_and_move(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """kernel.py:544-549."""
    if t.device.type == "cuda":
        return t
    if device.type != "cuda":
        raise RuntimeError("CUDA is required to run this kernel; no CUDA device available.")
    return t.to(device, non_blocking=True)


def _ensure_cuda(*tensors) -> torch.device:
    """kernel.py:552-559 (torch's "cuda" device is the HIP device on ROCm)."""
    if not torch.cuda.is_available():
        for t in tensors:
            if isinstance(t, torch.Tensor) and t.is_cuda:
                raise RuntimeError("CUDA inputs provided but CUDA is reported unavailable.")
        raise RuntimeError("CUDA is required to run this kernel; no CUDA device available.")
    return torch.device("cuda")


def _aligned(t: torch.Tensor, n: int) -> torch.Tensor:
    """t itself when its data is n-byte aligned (the kernels' widest access to it), else a copy
    (a fresh allocation is always aligned). The reference takes any tensor; this keeps that."""
    return t if t.data_ptr() % n == 0 else t.clone()


def validate(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
             gemm1_weights_scale, gemm2_weights, gemm2_weights_scale) -> int:
    """The dtype and shape checks of kernel.py:591-607; returns T."""
    assert hidden_states.dtype == torch.float8_e4m3fn, "hidden_states must be FLOAT8_E4M3FN"
    assert gemm1_weights.dtype == torch.float8_e4m3fn, "gemm1_weights must be FLOAT8_E4M3FN"
    assert gemm2_weights.dtype == torch.float8_e4m3fn, "gemm2_weights must be FLOAT8_E4M3FN"
    assert routing_logits.dtype == torch.float32, "routing_logits must be float32"
    assert routing_bias.dtype in (torch.float32, torch.bfloat16, torch.float16), \
        "routing_bias must be float or bf16/fp16"
    assert hidden_states_scale.dtype == torch.float32, "hidden_states_scale must be float32"
    assert gemm1_weights_scale.dtype == torch.float32, "gemm1_weights_scale must be float32"
    assert gemm2_weights_scale.dtype == torch.float32, "gemm2_weights_scale must be float32"

    T = int(routing_logits.shape[0])
    assert routing_logits.shape[-1] == EXPERTS_GLOBAL, "routing_logits last dim must be 256"
    assert hidden_states.shape == (T, HIDDEN), "hidden_states must be [T, 7168]"
    assert hidden_states_scale.shape == (H_BLOCKS, T), "hidden_states_scale must be [56, T]"
    assert gemm1_weights.shape == (EXPERTS_LOCAL, 2 * INTER, HIDDEN), "gemm1_weights must be [32, 4096, 7168]"
    assert gemm1_weights_scale.shape == (EXPERTS_LOCAL, G1_BLOCKS, H_BLOCKS), \
        "gemm1_weights_scale must be [32, 32, 56]"
    assert gemm2_weights.shape == (EXPERTS_LOCAL, HIDDEN, INTER), "gemm2_weights must be [32, 7168, 2048]"
    assert gemm2_weights_scale.shape == (EXPERTS_LOCAL, H_BLOCKS, I_BLOCKS), \
        "gemm2_weights_scale must be [32, 56, 16]"
    return T


class Workspace:
    """A device workspace for the C ABI, initialised once with moe_fp8_workspace_init.

    Every dispatch rewrites the control block before the GEMMs read it, so one workspace
    serves any number of successive calls issued on one stream. The initialisation is a
    kernel launch, so a workspace created while its stream is being captured into a graph
    puts a kernel node (never a memset node) into that graph.
    """

    def __init__(self, num_tokens: int, device: torch.device, stream: torch.cuda.Stream | None = None):
        self.layout = _lib.workspace_layout(num_tokens)
        self.nbytes = int(self.layout.total_bytes)
        self.buffer = torch.empty(max(self.nbytes, 256), dtype=torch.uint8, device=device)
        self.captured = False   # set once a graph capture has recorded a call using it
        # held while a call queues its kernels: calls from several host threads on one stream
        # (ctypes releases the GIL) then queue whole launch sequences one after another, so that
        # the kernels of two calls never interleave on the stream they share with the workspace
        self.lock = threading.Lock()
        stream = stream or torch.cuda.current_stream(device)
        _lib.check(_lib.load().moe_fp8_workspace_init(self.buffer.data_ptr(), self.buffer.numel(),
                                                      stream.cuda_stream), "moe_fp8_workspace_init")

    @property
    def ptr(self) -> int:
        return self.buffer.data_ptr()

    def view(self, name: str, dtype: torch.dtype, count: int) -> torch.Tensor:
        """The workspace array `name` (a moe_fp8_layout field) as a 1-D tensor of `count` items."""
        off = getattr(self.layout, name)
        nbytes = count * torch.empty((), dtype=dtype).element_size()
        return self.buffer[off:off + nbytes].view(dtype)


class WorkspaceCache:
    """One workspace per (device, stream), grown when a call needs more.

    A HIP graph that captured a call keeps that call's workspace pointer. A workspace that a
    capture has used is therefore never freed: when a larger call on its stream replaces it,
    it moves to a retired list that lives as long as the process, so that replays of the
    graph keep writing memory nobody else owns. Workspaces no capture has used are freed when
    replaced. A workspace created during a capture comes from the graph's memory pool and is
    kept alive here like any other. Replays and eager calls that share a workspace must not
    overlap in time: replay a graph on the stream it was captured on, or synchronise.

    `make(num_tokens, device, stream)` creates a workspace and `capturing()` says whether the
    current stream is being captured; both are injectable so that the policy is testable
    without a GPU.
    """

    def __init__(self, make=None, capturing=None):
        self._make = make or (lambda T, dev, stream: Workspace(T, dev, stream))
        self._capturing = capturing or torch.cuda.is_current_stream_capturing
        self._lock = threading.Lock()
        self._cache = {}
        self._retired = []

    def get(self, key, num_tokens: int, need_bytes: int, device, stream):
        with self._lock:
            ws = self._cache.get(key)
            if ws is None or ws.buffer.numel() < need_bytes:
                if ws is not None and ws.captured:
                    self._retired.append(ws)
                ws = self._make(num_tokens, device, stream)
                self._cache[key] = ws
            elif ws.layout.num_tokens != num_tokens:
                ws.layout = _lib.workspace_layout(num_tokens)
                ws.nbytes = int(ws.layout.total_bytes)
            if self._capturing():
                ws.captured = True
            return ws

    @property
    def retired(self) -> list:
        return list(self._retired)


_workspaces = WorkspaceCache()


def workspace_for(num_tokens: int, device: torch.device) -> Workspace:
    """The cached workspace of the current stream on `device`, grown to fit num_tokens."""
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    return _workspaces.get(key, num_tokens, _lib.workspace_bytes(num_tokens), device, stream)


class PackedWeightCache:
    """Packed copies of weight sets (pack_weights) that run() streams up to 256 tokens.

    The weights keep their kernel.py:604-607 contract: run() receives them row-major as ever,
    and the first call of up to 256 tokens with a weight set builds its packed copy (one kernel
    on the current stream, 1.41 GB), which later calls with the same set stream instead. A copy
    belongs to the weights' storage (W13's and W2's device addresses, held by weak reference) and
    to their version counters: modifying the weights in place through torch, or freeing them and
    allocating new ones at the same address, makes the copy stale, and the next call replaces it.
    Writes to the weights that bypass torch (raw pointers) are not seen: call clear() then.

    At most `max_sets` copies are held; further weight sets run on the row-major weights (no
    eviction, so that a model with more layers than copies never repacks in a loop). No copy is
    built while the current stream is being captured into a HIP graph; a copy that a capture has
    used is never freed (a stale one moves to a retired list), because the graph holds its
    address. A copy handed to a stream other than the one that built it is recorded on that
    stream (Tensor.record_stream), so that dropping a stale copy never lets the allocator reuse
    its memory while work queued on that stream may still read it, and that stream first waits
    for the event recorded right after the packing kernel: callers only read the weights and
    cannot know that a copy exists, so nothing else would order their stream after the build
    (under capture no wait is added: torch.cuda.graph synchronises the device before capturing,
    and a capture cannot wait on an event recorded outside it). A weight set whose copy does not
    fit in device memory (the allocation raises torch.cuda.OutOfMemoryError) runs on the
    row-major weights, and its copy is not tried again until clear(). `make(w13, w2)`,
    `capturing()`, `stream_id()`, `record(packed)`, `event()` (an event recorded on the current
    stream) and `wait(event)` are injectable so that the policy is testable without a GPU.
    """

    def __init__(self, max_sets: int = 4, make=None, capturing=None, storage_ref=None, stream_id=None,
                 record=None, event=None, wait=None):
        from torch.multiprocessing.reductions import StorageWeakRef
        self.max_sets = max_sets
        self._make = make or (lambda w13, w2: pack_weights(w13, w2))
        self._capturing = capturing or torch.cuda.is_current_stream_capturing
        self._ref = storage_ref or (lambda t: StorageWeakRef(t.untyped_storage()))
        self._stream_id = stream_id or (lambda: torch.cuda.current_stream().cuda_stream)
        self._record = record or (lambda packed: packed.record_stream(torch.cuda.current_stream(packed.device)))
        self._event = event or _record_event
        self._wait = wait or (lambda ev: torch.cuda.current_stream().wait_event(ev))
        self._lock = threading.Lock()
        self._entries = {}
        self._retired = []
        self._failed = set()   # weight sets whose copy did not fit in device memory

    def get(self, w13: torch.Tensor, w2: torch.Tensor):
        """The packed copy for (w13, w2), built if missing or stale; None when the set does
        not fit or the stream is being captured without a copy."""
        if self.max_sets <= 0:
            return None
        key = (w13.device.index, w13.data_ptr(), w2.data_ptr())
        version = (w13._version, w2._version)
        with self._lock:
            capturing = self._capturing()
            stream = self._stream_id()
            ent = self._entries.get(key)
            if ent is not None and not ent["ref13"].expired() and not ent["ref2"].expired() \
                    and ent["version"] == version:
                ent["captured"] = ent["captured"] or capturing
                if stream not in ent["streams"]:
                    self._record(ent["packed"])
                    if not capturing:
                        self._wait(ent["event"])   # the packing kernel before this stream's reads
                    ent["streams"].add(stream)
                return ent["packed"]
            if capturing or (key, version) in self._failed:
                return None
            if ent is not None:
                self._drop(key)
            for k in [k for k, v in self._entries.items() if v["ref13"].expired() or v["ref2"].expired()]:
                self._drop(k)
            if len(self._entries) >= self.max_sets:
                return None
            try:
                packed = self._make(w13, w2)
            except torch.cuda.OutOfMemoryError:
                self._failed.add((key, version))
                return None
            self._entries[key] = dict(ref13=self._ref(w13), ref2=self._ref(w2), version=version, packed=packed,
                                      captured=False, streams={stream}, event=self._event())
            return packed

    def _drop(self, key):
        ent = self._entries.pop(key)
        if ent["captured"]:
            self._retired.append(ent["packed"])

    def clear(self):
        """Forgets every copy (copies a graph capture used are kept alive in the retired list)."""
        with self._lock:
            for k in list(self._entries):
                self._drop(k)
            self._failed.clear()

    def __len__(self) -> int:
        return len(self._entries)

    @property
    def retired(self) -> list:
        return list(self._retired)


def _record_event():
    """An event recorded on the current stream (after the work queued there so far)."""
    ev = torch.cuda.Event()
    ev.record()
    return ev


_packed_weights = PackedWeightCache()


def packed_weights_for(gemm1_weights: torch.Tensor, gemm2_weights: torch.Tensor):
    """The packed copy run() uses for this weight set (built now if missing), or None when the
    cache is off or full."""
    return _packed_weights.get(gemm1_weights, gemm2_weights)


def clear_packed_weights() -> None:
    """Forgets run()'s packed copies (after writes to the weights that bypass torch); copies a
    graph capture used stay alive."""
    _packed_weights.clear()


def set_packed_weight_sets(max_sets: int) -> None:
    """How many weight sets run() keeps a packed copy of (default 4, 1.41 GB each); 0 turns the
    packed path of run() off. Copies already built are kept (see PackedWeightCache.clear)."""
    _packed_weights.max_sets = int(max_sets)


def make_args(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
              gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
              routed_scaling_factor, output) -> _lib.MoeFp8Args:
    """Packs device tensors into struct moe_fp8_args (pointers only; no copies)."""
    a = _lib.MoeFp8Args()
    a.routing_logits = routing_logits.data_ptr() if routing_logits is not None else None
    a.routing_bias = routing_bias.data_ptr() if routing_bias is not None else None
    a.routing_bias_dtype = _BIAS_CODES[routing_bias.dtype] if routing_bias is not None else BIAS_F32
    a.hidden_states = hidden_states.data_ptr()
    a.hidden_states_scale = hidden_states_scale.data_ptr()
    a.gemm1_weights = gemm1_weights.data_ptr()
    a.gemm1_weights_scale = gemm1_weights_scale.data_ptr()
    a.gemm2_weights = gemm2_weights.data_ptr()
    a.gemm2_weights_scale = gemm2_weights_scale.data_ptr()
    a.num_tokens = int(hidden_states.shape[0])
    a.local_expert_offset = int(local_expert_offset)
    a.routed_scaling_factor = float(routed_scaling_factor)
    a.output = output.data_ptr()
    a.output_dtype = OUT_F32 if output.dtype == torch.float32 else OUT_BF16
    return a


@torch.no_grad()
def run(
    routing_logits: torch.Tensor,
    routing_bias: torch.Tensor,
    hidden_states: torch.Tensor,
    hidden_states_scale: torch.Tensor,
    gemm1_weights: torch.Tensor,
    gemm1_weights_scale: torch.Tensor,
    gemm2_weights: torch.Tensor,
    gemm2_weights_scale: torch.Tensor,
    local_expert_offset: int,
    routed_scaling_factor: float,
    output: torch.Tensor,
):
    """The fused FP8 block-scale DeepSeek-V3 MoE layer; writes `output` in place.

    Same contract as kernel.py:562-729: inputs are validated with the reference's
    assertions, CPU inputs are moved to the GPU, and the result (the local experts'
    contribution, weighted by the renormalised routing weights) is written into
    `output` [T, 7168]. A bf16 or fp32 `output` on the GPU is written directly by the
    kernels; any other dtype or device receives a copy_ of a bf16 result.

    Up to 256 tokens, with contiguous weights already on the GPU, the GEMMs stream a packed copy
    of the weight set that the first such call builds and later calls reuse (PackedWeightCache;
    set_packed_weight_sets(0) turns it off). The output is bit-identical either way.
    """
    _run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
         gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor, output, _AUTO)
    return None


_AUTO = object()   # run(): the packed copy from the cache, when one applies


@torch.no_grad()
def pack_weights(gemm1_weights: torch.Tensor, gemm2_weights: torch.Tensor) -> torch.Tensor:
    """The packed copy of W13 and W2 that the decode GEMMs stream (moe_fp8_pack_weights): a uint8
    tensor of moe_fp8_packed_weights_bytes() on the weights' device, to be kept with the weight
    set and passed to run_packed. The weights keep their kernel.py:604-607 contract."""
    assert gemm1_weights.dtype == torch.float8_e4m3fn and tuple(gemm1_weights.shape) == (EXPERTS_LOCAL, 2 * INTER, HIDDEN), \
        "gemm1_weights must be float8_e4m3fn [32, 4096, 7168]"
    assert gemm2_weights.dtype == torch.float8_e4m3fn and tuple(gemm2_weights.shape) == (EXPERTS_LOCAL, HIDDEN, INTER), \
        "gemm2_weights must be float8_e4m3fn [32, 7168, 2048]"
    if not (gemm1_weights.is_cuda and gemm2_weights.is_cuda) or gemm1_weights.device != gemm2_weights.device:
        raise RuntimeError("pack_weights needs both weight tensors on one GPU")
    dev = gemm1_weights.device
    lib = _lib.load()
    w13, w2 = _aligned(gemm1_weights.contiguous(), 16), _aligned(gemm2_weights.contiguous(), 16)
    packed = torch.empty(_lib.packed_weights_bytes(), dtype=torch.uint8, device=dev)
    args = _lib.MoeFp8Args()
    args.gemm1_weights = w13.data_ptr()
    args.gemm2_weights = w2.data_ptr()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(lib.moe_fp8_pack_weights(args, packed.data_ptr(), packed.numel(), stream),
                   "moe_fp8_pack_weights")
    return packed


@torch.no_grad()
def run_packed(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
               gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset: int,
               routed_scaling_factor: float, output: torch.Tensor, *, packed_weights: torch.Tensor):
    """run() with the packed copy of this weight set (pack_weights): up to 256 tokens the GEMMs
    stream `packed_weights` instead of gemm1_weights / gemm2_weights; the output is bit-identical
    to run()'s."""
    assert packed_weights.dtype == torch.uint8 and packed_weights.is_contiguous() and \
        packed_weights.numel() >= _lib.packed_weights_bytes(), "packed_weights must come from pack_weights"
    _run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
         gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor, output, packed_weights)
    return None


def _run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
         gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor, output, packed):
    T = validate(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                 gemm1_weights_scale, gemm2_weights, gemm2_weights_scale)
    assert tuple(output.shape) == (T, HIDDEN), "output must be [T, 7168]"
    device = _ensure_cuda(routing_logits, routing_bias, hidden_states, hidden_states_scale,
                          gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale)
    lib = _lib.load()

    logits = _aligned(_check_cuda_and_move(routing_logits, device).contiguous(), 16)
    bias = _aligned(_check_cuda_and_move(routing_bias, device).contiguous(), 4)
    hidden = _aligned(_check_cuda_and_move(hidden_states, device).contiguous(), 16)
    hidden_scale = _aligned(_check_cuda_and_move(hidden_states_scale, device).contiguous(), 4)
    w13 = _aligned(_check_cuda_and_move(gemm1_weights, device).contiguous(), 16)
    w13_scale = _aligned(_check_cuda_and_move(gemm1_weights_scale, device).contiguous(), 4)
    w2 = _aligned(_check_cuda_and_move(gemm2_weights, device).contiguous(), 16)
    w2_scale = _aligned(_check_cuda_and_move(gemm2_weights_scale, device).contiguous(), 4)
    dev = logits.device
    for t in (bias, hidden, hidden_scale, w13, w13_scale, w2, w2_scale):
        if t.device != dev:
            raise RuntimeError(f"all inputs must be on one device; got {t.device} and {dev}")

    direct = output.is_cuda and output.device == dev and output.is_contiguous() and \
        output.dtype in (torch.bfloat16, torch.float32) and output.data_ptr() % 16 == 0
    dst = output if direct else torch.empty((T, HIDDEN), dtype=torch.bfloat16, device=dev)
    if T == 0:
        return None
    with torch.cuda.device(dev):
        ws = workspace_for(T, dev)
        args = make_args(logits, bias, hidden, hidden_scale, w13, w13_scale, w2, w2_scale,
                         local_expert_offset, routed_scaling_factor, dst)
        stream = torch.cuda.current_stream(dev).cuda_stream
        if packed is _AUTO:
            packed = _packed_weights.get(w13, w2) if (
                T <= PACKED_MAX_TOKENS and w13 is gemm1_weights and w2 is gemm2_weights) else None
        if packed is not None and packed.device != dev:
            raise RuntimeError(f"packed_weights must be on {dev}; got {packed.device}")
        with ws.lock:
            if packed is None:
                _lib.check(lib.moe_fp8_run(args, ws.ptr, ws.buffer.numel(), stream), "moe_fp8_run")
            else:
                _lib.check(lib.moe_fp8_run_packed(args, packed.data_ptr(), packed.numel(), ws.ptr,
                                                  ws.buffer.numel(), stream), "moe_fp8_run_packed")
    if not direct:
        output.copy_(dst)


_HIDDEN_CODES = {torch.float32: HIDDEN_F32, torch.bfloat16: HIDDEN_BF16, torch.float16: HIDDEN_F16}


@torch.no_grad()
def quantize_hidden(hidden: torch.Tensor, out: torch.Tensor | None = None,
                    out_scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The step before `run`: hidden states [T, 7168] (bf16, fp16 or fp32) to the layer's
    activation contract (kernel.py:600-603): e4m3fn [T, 7168] and fp32 scales [56, T],
    per token and 128-column block scale = max(amax / 448, 1e-12), q = e4m3(x / scale)
    rounded to nearest even (the reference's in-path requantisation, kernel.py:131-135).

    Returns (hidden_states, hidden_states_scale), written into `out` / `out_scale` when
    given (contiguous tensors of those shapes and dtypes on the input's GPU).
    """
    assert hidden.dtype in _HIDDEN_CODES, "hidden must be float32, bfloat16 or float16"
    assert hidden.dim() == 2 and hidden.shape[1] == HIDDEN, "hidden must be [T, 7168]"
    device = _ensure_cuda(hidden, out, out_scale)
    x = _aligned(_check_cuda_and_move(hidden, device).contiguous(), 16)
    T = int(x.shape[0])
    if out is None:
        out = torch.empty((T, HIDDEN), dtype=torch.float8_e4m3fn, device=x.device)
    if out_scale is None:
        out_scale = torch.empty((H_BLOCKS, T), dtype=torch.float32, device=x.device)
    assert out.dtype == torch.float8_e4m3fn and tuple(out.shape) == (T, HIDDEN), "out must be float8_e4m3fn [T, 7168]"
    assert out_scale.dtype == torch.float32 and tuple(out_scale.shape) == (H_BLOCKS, T), \
        "out_scale must be float32 [56, T]"
    for t in (out, out_scale):
        if not (t.is_cuda and t.device == x.device and t.is_contiguous()):
            raise RuntimeError("out and out_scale must be contiguous tensors on the input's device")
    if T == 0:
        return out, out_scale
    # destinations the kernel cannot store to directly (8-byte fp8 stores, 4-byte scale stores)
    # are written through aligned temporaries
    q = out if out.data_ptr() % 8 == 0 else torch.empty_like(out)
    qs = out_scale if out_scale.data_ptr() % 4 == 0 else torch.empty_like(out_scale)
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.load().moe_fp8_quantize_hidden(x.data_ptr(), _HIDDEN_CODES[x.dtype], T, q.data_ptr(),
                                                       qs.data_ptr(), stream), "moe_fp8_quantize_hidden")
    if q is not out:
        out.copy_(q)
    if qs is not out_scale:
        out_scale.copy_(qs)
    return out, out_scale
