"""Python binding of the MI355X sampler C ABI (include/nimbus_sampler.h).

Mirrors the reference's `nimbus_infer_rs::sampler` module (src/sampler.rs):
`SamplingParams`, `Rng`, `sample()`, plus the batched device entry point
`Sampler.sample_batch()` over [B, V] fp32 logits already resident in HBM.
PyTorch is used only for device memory and the current HIP stream.

There is no CPU fallback: if the HIP library is missing or fails to load,
every entry point raises.
"""
import ctypes
import dataclasses
import os
from typing import List, Optional, Sequence

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(ROOT_DIR, "lib", "libnimbus_sampler.so")

NIS_OK, NIS_EINVAL, NIS_ERANGE, NIS_EALIGN, NIS_ENODEV = 0, -1, -2, -3, -4
NIS_MAX_V = 1 << 20
PATH_GREEDY, PATH_NONFINITE_MAX, PATH_BAD_TOTAL, PATH_DRAW, PATH_FALLTHROUGH = 1, 2, 3, 4, 5

# nis_row_stats
ROW_STATS_DTYPE = np.dtype([
    ("max_w", "<f8"), ("z_kept", "<f8"), ("z_all", "<f8"), ("u", "<f8"), ("prob", "<f8"),
    ("kept", "<u8"), ("path", "<u4"), ("token", "<u4"), ("kernel", "<u4"), ("reject", "<u4"),
])
assert ROW_STATS_DTYPE.itemsize == 64

EXPORTED_SYMBOLS = (
    "nis_ctx_create", "nis_ctx_destroy", "nis_ctx_set_stream", "nis_ctx_get_stream",
    "nis_last_error", "nis_status_string", "nis_rng_seed", "nis_rng_next_u64",
    "nis_rng_next_f64", "nis_rng_seed_batch", "nis_sample_batch", "nis_argmax_batch",
    "nis_apply_repetition_penalty", "nis_sample_one", "nis_sample_one_noalloc", "nis_sync",
    "nis_decode_step",
    "nis_lm_head_logits", "nis_lm_head_greedy", "nis_stream_floor", "nis_stream_floor_split",
)


class NisParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("reserved", ctypes.c_uint32),
                ("top_k", ctypes.c_uint64)]


W_F32, W_INT8, W_INT4 = 0, 8, 4


class NisWeights(ctypes.Structure):
    """nis_weights: format, group size (0 = per row), data and scales pointers."""
    _fields_ = [("format", ctypes.c_int32), ("group_size", ctypes.c_int32),
                ("d_data", ctypes.c_void_p), ("d_scales", ctypes.c_void_p)]


class SamplerError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"nimbus sampler error {status}: {message}")
        self.status = status


_lib = None


def load_library(path: str = LIB_PATH):
    """Load libnimbus_sampler.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SamplerError(NIS_EINVAL, f"{path} not built (run __graft_entry__.build())")
    # torch bundles its own libamdhip64.so.7 (same SONAME as /opt/rocm's).
    # Initialise torch's HIP runtime first so the library binds to that one
    # copy: device pointers and streams are then shared with torch tensors.
    try:
        import torch
        if torch.cuda.is_available():
            torch.cuda.init()
    except ImportError:
        pass
    L = ctypes.CDLL(path)
    vp, u64p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)
    L.nis_ctx_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
    L.nis_ctx_destroy.argtypes = [vp]
    L.nis_ctx_set_stream.argtypes = [vp, vp]
    L.nis_ctx_get_stream.argtypes = [vp]
    L.nis_ctx_get_stream.restype = vp
    L.nis_last_error.argtypes = [vp]
    L.nis_last_error.restype = ctypes.c_char_p
    L.nis_status_string.argtypes = [ctypes.c_int]
    L.nis_status_string.restype = ctypes.c_char_p
    L.nis_rng_seed.argtypes = [ctypes.c_uint64, u64p]
    L.nis_rng_next_u64.argtypes = [u64p]
    L.nis_rng_next_u64.restype = ctypes.c_uint64
    L.nis_rng_next_f64.argtypes = [u64p]
    L.nis_rng_next_f64.restype = ctypes.c_double
    L.nis_rng_seed_batch.argtypes = [vp, vp, ctypes.c_int32, vp]
    L.nis_sample_batch.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.POINTER(NisParams), vp, vp, vp, vp, vp]
    L.nis_argmax_batch.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64, vp]
    L.nis_decode_step.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                  ctypes.POINTER(NisParams), vp, vp, ctypes.c_int64, vp, vp, vp,
                                  ctypes.c_int32, vp, vp, vp]
    L.nis_lm_head_logits.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.POINTER(NisWeights), ctypes.c_int64, vp, ctypes.c_int64]
    L.nis_lm_head_greedy.argtypes = [vp, vp, ctypes.c_int32, ctypes.POINTER(NisWeights),
                                     ctypes.c_int64, vp, vp]
    L.nis_apply_repetition_penalty.argtypes = [vp, vp, ctypes.c_int64, vp, ctypes.c_int64,
                                               ctypes.c_float]
    L.nis_sample_one.argtypes = [vp, vp, ctypes.c_int64, ctypes.POINTER(NisParams), vp,
                                 ctypes.c_int64, u64p, ctypes.POINTER(ctypes.c_uint32)]
    L.nis_sample_one_noalloc.argtypes = L.nis_sample_one.argtypes
    L.nis_sync.argtypes = [vp]
    L.nis_stream_floor.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_float, vp]
    L.nis_stream_floor_split.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                         ctypes.c_float, ctypes.c_int32, vp, vp]
    for name in ("nis_ctx_create", "nis_ctx_destroy", "nis_ctx_set_stream", "nis_rng_seed_batch",
                 "nis_sample_batch", "nis_argmax_batch", "nis_apply_repetition_penalty",
                 "nis_sample_one", "nis_sample_one_noalloc", "nis_sync", "nis_stream_floor",
                 "nis_stream_floor_split"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


# ---------------------------------------------------------------------------
# Reference API mirror (src/sampler.rs)

@dataclasses.dataclass
class SamplingParams:
    """SamplingParams (sampler.rs:6-35) with the reference defaults."""
    max_new_tokens: int = 64
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    seed: Optional[int] = None
    stop_tokens: List[int] = dataclasses.field(default_factory=list)

    def greedy(self) -> bool:
        return np.float32(self.temperature) <= 0.0

    def to_c(self) -> NisParams:
        return NisParams(float(np.float32(self.temperature)), float(np.float32(self.top_p)),
                         float(np.float32(self.repetition_penalty)), 0, int(self.top_k))


class Rng:
    """Rng (sampler.rs:40-78): xoshiro256++ seeded by SplitMix64, host-held
    32-byte state that crosses the ABI as four u64 words."""

    def __init__(self, seed: int):
        self._s = (ctypes.c_uint64 * 4)()
        load_library().nis_rng_seed(ctypes.c_uint64(int(seed) & (2**64 - 1)), self._s)

    @classmethod
    def from_state(cls, words: Sequence[int]) -> "Rng":
        r = cls.__new__(cls)
        r._s = (ctypes.c_uint64 * 4)(*[int(w) & (2**64 - 1) for w in words])
        return r

    def state(self) -> List[int]:
        return [int(v) for v in self._s]

    def next_u64(self) -> int:
        return int(load_library().nis_rng_next_u64(self._s))

    def next_f64(self) -> float:
        return float(load_library().nis_rng_next_f64(self._s))


def rng_states(seeds: Sequence[int]) -> np.ndarray:
    """[B,4] uint64 host array of Rng::new(seed) states."""
    out = np.zeros((len(seeds), 4), dtype=np.uint64)
    for i, s in enumerate(seeds):
        out[i] = Rng(int(s)).state()
    return out


def _check(L, ctx, rc):
    if rc != NIS_OK:
        msg = L.nis_last_error(ctx) if ctx else None
        msg = msg.decode() if msg else L.nis_status_string(rc).decode()
        raise SamplerError(rc, msg)


class Sampler:
    """A sampler context (one device, launches on torch's current stream)."""

    def __init__(self, device: int = 0):
        L = load_library()
        self._L = L
        self._ctx = ctypes.c_void_p()
        _check(L, None, L.nis_ctx_create(int(device), ctypes.byref(self._ctx)))
        self.device = device

    def close(self):
        if self._ctx:
            self._L.nis_ctx_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._ctx

    def _bind_stream(self):
        import torch
        self._L.nis_ctx_set_stream(self._ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    def sample_batch(self, logits, params: SamplingParams, rng_states, V: Optional[int] = None,
                     gen_ids=None, gen_offsets=None, tokens=None, stats=None):
        """Batched sample() on device tensors.

        logits: float32 [B, ld] (row stride ld >= V, unit column stride);
        rng_states: int64 [B, 4] holding the u64 words, advanced in place;
        gen_ids: int32 [n] / gen_offsets: int64 [B+1] CSR history (optional);
        tokens: optional int32 [B] output; stats: optional uint8 [B, 64].
        Returns the tokens tensor.  Asynchronous on torch's current stream."""
        import torch
        assert logits.dtype == torch.float32 and logits.dim() == 2 and logits.stride(1) == 1
        B = logits.shape[0]
        V = logits.shape[1] if V is None else V
        if tokens is None:
            tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
        self._bind_stream()
        p = params.to_c() if isinstance(params, SamplingParams) else params
        rc = self._L.nis_sample_batch(
            self._ctx, ctypes.c_void_p(logits.data_ptr()), logits.stride(0), B, V, ctypes.byref(p),
            ctypes.c_void_p(rng_states.data_ptr()) if rng_states is not None else None,
            ctypes.c_void_p(gen_ids.data_ptr()) if gen_ids is not None else None,
            ctypes.c_void_p(gen_offsets.data_ptr()) if gen_offsets is not None else None,
            ctypes.c_void_p(tokens.data_ptr()),
            ctypes.c_void_p(stats.data_ptr()) if stats is not None else None)
        _check(self._L, self._ctx, rc)
        return tokens

    def decode_step(self, logits, params: SamplingParams, rng_states, gen_ids, gen_len, max_new,
                    done, stop_ids=None, V: Optional[int] = None, tokens=None, stats=None):
        """One step of a batched decode loop (engine.rs:279-287) on device tensors.

        gen_ids: int32 [B, cap] histories (also the penalty lists), gen_len:
        int32 [B], max_new: int32 [B], done: uint8 [B], stop_ids: int32 [n]
        (optional).  Sequences not yet done sample a token, append it and may
        finish; done ones are skipped.  Returns the tokens tensor."""
        import torch
        assert logits.dtype == torch.float32 and logits.dim() == 2 and logits.stride(1) == 1
        assert gen_ids.dim() == 2 and gen_ids.stride(1) == 1
        B = logits.shape[0]
        V = logits.shape[1] if V is None else V
        if tokens is None:
            tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
        self._bind_stream()
        p = params.to_c() if isinstance(params, SamplingParams) else params
        n_stop = 0 if stop_ids is None else int(stop_ids.numel())
        rc = self._L.nis_decode_step(
            self._ctx, ctypes.c_void_p(logits.data_ptr()), logits.stride(0), B, V, ctypes.byref(p),
            ctypes.c_void_p(rng_states.data_ptr()) if rng_states is not None else None,
            ctypes.c_void_p(gen_ids.data_ptr()), gen_ids.stride(0),
            ctypes.c_void_p(gen_len.data_ptr()), ctypes.c_void_p(max_new.data_ptr()),
            ctypes.c_void_p(stop_ids.data_ptr()) if n_stop else None, n_stop,
            ctypes.c_void_p(done.data_ptr()), ctypes.c_void_p(tokens.data_ptr()),
            ctypes.c_void_p(stats.data_ptr()) if stats is not None else None)
        _check(self._L, self._ctx, rc)
        return tokens

    def _weights(self, H: int, fmt: int, data, V: int, scales, group_size: int, tensors):
        """nis_weights for a [V, H] head, after checking every size the C ABI
        will read (it sees bare pointers) and that all tensors share the
        sampler's device."""
        import torch
        fmt, group_size = int(fmt), int(group_size)
        if fmt == W_F32:
            need, ddtype = V * H, torch.float32
        elif fmt == W_INT8:
            need, ddtype = V * H, torch.uint8
        elif fmt == W_INT4:
            need, ddtype = (V * H + 1) // 2, torch.uint8
        else:
            raise SamplerError(NIS_EINVAL, f"unknown weight format {fmt}")
        if data.dtype != ddtype or not data.is_contiguous() or data.numel() < need:
            raise SamplerError(NIS_EINVAL, f"weights must be contiguous {ddtype} with at least "
                                           f"{need} elements (got {data.dtype}, {data.numel()})")
        tensors = list(tensors) + [data]
        if fmt != W_F32:
            groups = H // group_size if group_size > 0 and H % group_size == 0 else 1
            if scales is None or scales.dtype != torch.float32 or not scales.is_contiguous() or \
                    scales.numel() < V * groups:
                raise SamplerError(NIS_EINVAL, f"scales must be contiguous float32 with at least "
                                               f"{V * groups} elements")
            tensors.append(scales)
        dev = torch.device("cuda", self.device)
        if any(t.device != dev for t in tensors):
            raise SamplerError(NIS_EINVAL, f"hidden, weights, scales and outputs must be on {dev}")
        return NisWeights(fmt, group_size, data.data_ptr(),
                          scales.data_ptr() if scales is not None else None)

    def lm_head_logits(self, hidden, fmt: int, data, V: int, scales=None, group_size: int = 0,
                       out=None):
        """Logits of B last-hidden rows (model.rs:317-325) on device tensors.

        hidden: float32 [B, ldh] (unit column stride); data: the weights —
        float32 [V, H] (W_F32), uint8 [V, H] biased codes (W_INT8) or uint8
        [ceil(V*H/2)] packed nibbles (W_INT4); scales: float32 [V] or
        [V, H/group_size].  out: optional float32 [B, ld >= V].  Returns out."""
        import torch
        assert hidden.dtype == torch.float32 and hidden.dim() == 2 and hidden.stride(1) == 1
        B = hidden.shape[0]
        H = hidden.shape[1]
        if out is None:
            out = torch.empty((B, V), dtype=torch.float32, device=hidden.device)
        if out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1 or \
                out.shape[0] < B or out.shape[1] < V:
            raise SamplerError(NIS_EINVAL, "out must be float32 [>= B, >= V] with unit column stride")
        w = self._weights(H, fmt, data, V, scales, group_size, [hidden, out])
        self._bind_stream()
        rc = self._L.nis_lm_head_logits(self._ctx, ctypes.c_void_p(hidden.data_ptr()),
                                        hidden.stride(0), B, H, ctypes.byref(w), V,
                                        ctypes.c_void_p(out.data_ptr()), out.stride(0))
        _check(self._L, self._ctx, rc)
        return out

    def lm_head_greedy(self, hidden, fmt: int, data, V: int, scales=None, group_size: int = 0,
                       logits=None, token=None):
        """Greedy token of one last-hidden row (model.rs:317-325, then
        sampler.rs:172-181) in one pass over the head (nis_lm_head_greedy).

        hidden: float32 [H] or [1, H]; logits: optional float32 [>= V] that
        also receives the logits; token: optional int32 [1].  Returns token."""
        import torch
        h = hidden.reshape(-1)
        assert h.dtype == torch.float32 and h.is_contiguous()
        H = h.numel()
        if token is None:
            token = torch.empty(1, dtype=torch.int32, device=h.device)
        if token.dtype != torch.int32 or token.numel() < 1:
            raise SamplerError(NIS_EINVAL, "token must be int32 with one element")
        tensors = [h, token]
        if logits is not None:
            if logits.dtype != torch.float32 or not logits.is_contiguous() or logits.numel() < V:
                raise SamplerError(NIS_EINVAL, "logits must be contiguous float32 [>= V]")
            tensors.append(logits)
        w = self._weights(H, fmt, data, V, scales, group_size, tensors)
        self._bind_stream()
        rc = self._L.nis_lm_head_greedy(
            self._ctx, ctypes.c_void_p(h.data_ptr()), H, ctypes.byref(w), V,
            ctypes.c_void_p(logits.data_ptr()) if logits is not None else None,
            ctypes.c_void_p(token.data_ptr()))
        _check(self._L, self._ctx, rc)
        return token

    def argmax_batch(self, logits, V: Optional[int] = None, tokens=None):
        import torch
        B = logits.shape[0]
        V = logits.shape[1] if V is None else V
        if tokens is None:
            tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
        self._bind_stream()
        rc = self._L.nis_argmax_batch(self._ctx, ctypes.c_void_p(logits.data_ptr()),
                                      logits.stride(0), B, V, ctypes.c_void_p(tokens.data_ptr()))
        _check(self._L, self._ctx, rc)
        return tokens

    def stream_floor(self, logits, temperature: float, V: Optional[int] = None, out=None):
        """Measurement only (nis_stream_floor): each row's max and sum of
        2^(x c - ceil(max c)) read with the sparse kernel's layout; out is a
        [B, 2] float32 tensor.  Samples nothing."""
        import torch
        B = logits.shape[0]
        V = logits.shape[1] if V is None else V
        if out is None:
            out = torch.empty((B, 2), dtype=torch.float32, device=logits.device)
        self._bind_stream()
        rc = self._L.nis_stream_floor(self._ctx, ctypes.c_void_p(logits.data_ptr()),
                                      logits.stride(0), B, V, ctypes.c_float(temperature),
                                      ctypes.c_void_p(out.data_ptr()))
        _check(self._L, self._ctx, rc)
        return out

    def stream_floor_split(self, logits, temperature: float, S: int, V: Optional[int] = None,
                           out=None, part=None):
        """Measurement only (nis_stream_floor_split): stream_floor's result
        with each row read by S workgroups and their per-wave partials merged
        by a second launch; part is a [B * S * 4, 4] float32 workspace."""
        import torch
        B = logits.shape[0]
        V = logits.shape[1] if V is None else V
        if out is None:
            out = torch.empty((B, 2), dtype=torch.float32, device=logits.device)
        if part is None:
            part = torch.empty((B * S * 4, 4), dtype=torch.float32, device=logits.device)
        self._bind_stream()
        rc = self._L.nis_stream_floor_split(self._ctx, ctypes.c_void_p(logits.data_ptr()),
                                            logits.stride(0), B, V, ctypes.c_float(temperature), S,
                                            ctypes.c_void_p(part.data_ptr()),
                                            ctypes.c_void_p(out.data_ptr()))
        _check(self._L, self._ctx, rc)
        return out

    def rng_seed_batch(self, seeds, states):
        self._bind_stream()
        rc = self._L.nis_rng_seed_batch(self._ctx, ctypes.c_void_p(seeds.data_ptr()),
                                        seeds.numel(), ctypes.c_void_p(states.data_ptr()))
        _check(self._L, self._ctx, rc)
        return states

    def apply_repetition_penalty(self, logits_f64, generated, penalty: float):
        self._bind_stream()
        rc = self._L.nis_apply_repetition_penalty(
            self._ctx, ctypes.c_void_p(logits_f64.data_ptr()), logits_f64.numel(),
            ctypes.c_void_p(generated.data_ptr()) if generated.numel() else None,
            generated.numel(), ctypes.c_float(penalty))
        _check(self._L, self._ctx, rc)
        return logits_f64

    def sample_one(self, logits, params: SamplingParams, generated: Sequence[int], rng: Rng) -> int:
        """Host-buffer drop-in of sample(&logits, params, &generated, &mut rng)."""
        x = np.ascontiguousarray(logits, dtype=np.float32)
        g = np.ascontiguousarray(generated, dtype=np.uint32)
        tok = ctypes.c_uint32()
        p = params.to_c()
        rc = self._L.nis_sample_one(self._ctx, ctypes.c_void_p(x.ctypes.data), x.size,
                                    ctypes.byref(p), ctypes.c_void_p(g.ctypes.data) if g.size else None,
                                    g.size, rng._s, ctypes.byref(tok))
        _check(self._L, self._ctx, rc)
        return int(tok.value)

    def sync(self):
        _check(self._L, self._ctx, self._L.nis_sync(self._ctx))


_default_sampler: Optional[Sampler] = None


def sample(logits, params: SamplingParams, generated: Sequence[int], rng: Rng) -> int:
    """sample(logits, params, generated, rng) -> u32 (sampler.rs:163-168), on the GPU."""
    global _default_sampler
    if _default_sampler is None:
        _default_sampler = Sampler(int(os.environ.get("NIMBUS_DEVICE", "0")))
    return _default_sampler.sample_one(logits, params, generated, rng)


def stats_view(stats_u8) -> np.ndarray:
    """Host structured view of a uint8 [B, 64] stats tensor."""
    return np.ascontiguousarray(stats_u8.cpu().numpy()).view(ROW_STATS_DTYPE).reshape(-1)
