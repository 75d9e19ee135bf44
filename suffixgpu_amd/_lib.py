"""ctypes binding of the C ABI in include/suffixgpu_amd.h.

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing, or a tensor is not on a ROCm GPU, the call
raises.  Every entry point is enqueued on the caller's current HIP stream
(``torch.cuda.current_stream().cuda_stream``), so the whole drafter step
can be captured into a HIP graph.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsuffixgpu_amd.so"
MAX_CANDIDATES = 32
ABI_VERSION = 15

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_p = ctypes.c_void_p


class SfxParams(ctypes.Structure):
    _fields_ = [
        ("k", c_i32), ("max_pattern_len", c_i32), ("max_occurrences", c_i32),
        ("min_match_len", c_i32), ("num_thresholds", c_i32),
        ("num_caps", c_i32), ("has_spec_factor", c_i32),
        ("spec_factor", ctypes.c_float), ("spec_offset", ctypes.c_float),
        ("min_token_prob", ctypes.c_float), ("alpha", ctypes.c_float),
        ("thresholds", c_i32 * MAX_CANDIDATES),
        ("caps", c_i32 * MAX_CANDIDATES),
    ]


class SfxIndex(ctypes.Structure):
    _fields_ = [
        ("corpus", c_p), ("sa", c_p), ("capacity", c_i64),
        ("delta", c_p), ("delta_capacity", c_i64), ("delta_len", c_p),
        ("sa_key", c_p), ("key_width", c_i64),
        ("sa_key_alt", c_p), ("key_select", c_p),
        ("gram", c_p), ("gram_alt", c_p), ("gram_slots", c_i64),
        ("delta_entries", c_p), ("delta_start", c_p),
        ("delta_buckets", c_i64),
    ]


class SfxBatch(ctypes.Structure):
    _fields_ = [
        ("tokens", c_p), ("batch", c_i64), ("seq", c_i64),
        ("num_tokens", c_p), ("num_tokens_is64", c_i32),
        ("sampled", c_p), ("num_sampled", c_i64),
        ("valid_count", c_p), ("valid_count_is64", c_i32),
        ("mask", c_p), ("limit", c_i64),
    ]


class SfxGlobalOut(ctypes.Structure):
    _fields_ = [(name, c_p) for name in (
        "sa_len", "sa_start", "sa_end", "d_len", "d_pos", "d_cnt",
        "len", "cont", "occ", "draft", "emit", "draft_len", "draft_occ",
        "draft_score")]


class SfxAppendDoc(ctypes.Structure):
    _fields_ = [("src", c_p), ("n", c_i64), ("dst", c_i64)]


APPEND_MAX_DOCS = 64

# name -> (restype, argtypes)
SIGNATURES = {
    "sfx_abi_version": (c_i32, []),
    "sfx_sa_build_rounds_total": (c_i32, [c_i64]),
    "sfx_sa_build_flag_offset": (c_i64, [c_i64]),
    "sfx_sa_group_cap": (c_i32, []),
    "sfx_sa_build_begin": (c_i32, [c_p, c_i64, c_p, ctypes.c_size_t, c_p]),
    "sfx_sa_build_rounds": (c_i32, [c_i64, c_i32, c_i32, c_i32, c_p,
                                    ctypes.c_size_t, c_p]),
    "sfx_sa_build_finish": (c_i32, [c_i64, c_i64, c_p, c_i32, c_p,
                                    ctypes.c_size_t, c_p]),
    "sfx_index_swap": (c_i32, [c_p, c_p, c_p, c_p, c_i64, c_p, c_i32, c_p]),
    "sfx_delta_append": (c_i32, [ctypes.POINTER(SfxAppendDoc), c_i32, c_p,
                                 c_i64, c_p, c_i64, c_p]),
    "sfx_delta_shift": (c_i32, [c_p, c_i64, c_i64, c_i64, c_p, c_p]),
    "sfx_ingest_layout": (c_i32, [c_i64, c_i64, c_p]),
    "sfx_ingest_docs": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_p, c_p,
                                c_p, c_i64, c_i64, c_p, c_i32, c_p, c_i32,
                                c_i64, c_i64, c_p]),
    "sfx_ingest_active": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_p, c_p,
                                  c_p, c_i64, c_i64, c_p, c_i32, c_p, c_i32,
                                  c_i64, c_p, c_i64, c_i32, c_i64, c_i64,
                                  c_i64, c_p]),
    "sfx_ingest_swapped": (c_i32, [c_p, c_p]),
    "sfx_scatter_append": (c_i32, [ctypes.POINTER(SfxBatch), c_p, c_p]),
    "sfx_match_back": (c_i32, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p,
                               c_p]),
    "sfx_first_occurrences": (c_i32, [c_p, c_i64, c_p, c_i64, c_i64, c_i64,
                                      c_p, c_p, c_p]),
    "sfx_sa_search": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_i64, c_p, c_p,
                              c_p, c_p]),
    "sfx_expand_chain": (c_i32, [c_p, c_i64, c_i64, c_i64, c_p, c_p, c_p,
                                 ctypes.c_float, ctypes.c_float, c_p, c_p,
                                 c_p, c_p, c_p]),
    "sfx_local_gather": (c_i32, [ctypes.POINTER(SfxParams),
                                 ctypes.POINTER(SfxBatch), c_p, c_p, c_p,
                                 c_p]),
    "sfx_local_forward": (c_i32, [ctypes.POINTER(SfxParams),
                                  ctypes.POINTER(SfxBatch), c_p, c_p, c_p,
                                  c_p, c_p, c_p]),
    "sfx_global_query_workspace_size": (ctypes.c_size_t,
                                        [ctypes.POINTER(SfxParams), c_i64,
                                         c_i64]),
    "sfx_global_query": (c_i32, [ctypes.POINTER(SfxParams),
                                 ctypes.POINTER(SfxIndex), c_p, c_i64, c_i64,
                                 c_p, ctypes.POINTER(SfxGlobalOut), c_p,
                                 ctypes.c_size_t, c_p]),
    "sfx_step_workspace_size": (ctypes.c_size_t,
                                [ctypes.POINTER(SfxParams), c_i64, c_i64]),
    "sfx_propose_step": (c_i32, [ctypes.POINTER(SfxParams),
                                 ctypes.POINTER(SfxIndex),
                                 ctypes.POINTER(SfxBatch), c_p, c_p, c_p,
                                 c_p, ctypes.c_size_t, c_p]),
    "sfx_propose_step_noalloc": (c_i32, [ctypes.POINTER(SfxParams),
                                         ctypes.POINTER(SfxIndex),
                                         ctypes.POINTER(SfxBatch), c_p, c_p,
                                         c_p, c_p]),
    "sfx_sa_build_workspace_size": (ctypes.c_size_t, [c_i64]),
    "sfx_sa_keys": (c_i32, [c_p, c_p, c_i64, c_i64, c_i64, c_p, c_p, c_p]),
    "sfx_gram_table_bytes": (ctypes.c_size_t, [c_i64]),
    "sfx_gram_build": (c_i32, [c_p, c_i64, c_i64, c_p, c_i64, c_p]),
    "sfx_delta_index_bytes": (ctypes.c_size_t, [c_i64]),
    "sfx_delta_index_build": (c_i32, [c_p, c_p, c_i64, c_p, c_p, c_i64, c_p,
                                      ctypes.c_size_t, c_p]),
    "sfx_sa_build": (c_i32, [c_p, c_i64, c_i64, c_p, c_i32, c_p,
                             ctypes.c_size_t, c_p]),
}

_lib = None


class SuffixGPUError(RuntimeError):
    pass


def _check_single_hip_runtime() -> None:
    """Refuse to run with two HIP runtimes mapped (torch's and ROCm's)."""
    try:
        maps = Path("/proc/self/maps").read_text()
    except OSError:
        return
    paths = {line.split()[-1] for line in maps.splitlines()
             if "libamdhip64" in line and "/" in line}
    if len({os.path.realpath(p) for p in paths}) > 1:
        raise SuffixGPUError(
            "two HIP runtimes are loaded (" + ", ".join(sorted(paths)) +
            "); the drafter library must share torch's runtime")


def lib() -> ctypes.CDLL:
    """Load the HIP library (once); raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise SuffixGPUError(
            f"{LIB_PATH} is missing: build it with "
            "`python -m suffixgpu_amd.build` (hipcc, gfx950)")
    import torch  # noqa: F401  (load torch's HIP runtime first)
    handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    if handle.sfx_abi_version() != ABI_VERSION:
        raise SuffixGPUError("libsuffixgpu_amd ABI version mismatch")
    _check_single_hip_runtime()
    _lib = handle
    return _lib


# Error codes of the C ABI besides hipError_t values.
EINVAL = -1
ENOSCRATCH = -2
NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_MAX_ROWS = 4096
# flags of sfx_sa_build_rounds
SA_ROUNDS_RADIX = 1
SA_ROUNDS_EXPECT_FINAL = 2
INGEST_MAX_DOCS = 4096
# sfx_ingest_header, in order (int64 each)
INGEST_HEADER_FIELDS = (
    "active_len", "live_active_len", "delta_len", "active_head",
    "active_docs", "delta_head", "delta_docs", "in_flight", "snap_seq",
    "snap_n_new", "snap_m", "docs_in", "docs_dropped", "tokens_dropped",
    "bad_rows", "reserved")


def check(rc: int, what: str) -> None:
    if rc != 0:
        if rc == EINVAL:
            raise SuffixGPUError(f"{what}: invalid argument")
        if rc == ENOSCRATCH:
            raise SuffixGPUError(
                f"{what}: the batch needs more than the "
                f"{NOALLOC_SCRATCH_BYTES >> 20} MiB static step scratch "
                f"(or more than {NOALLOC_MAX_ROWS} rows); use the "
                "workspace form")
        raise SuffixGPUError(f"{what}: HIP error {rc}")


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise SuffixGPUError(
                "suffixgpu_amd runs on ROCm GPU tensors only (got a "
                f"{t.device} tensor); there is no CPU path")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def make_params(k: int, max_pattern_len: int, max_occurrences: int,
                min_match_len: int, thresholds, caps,
                max_spec_factor: float | None, max_spec_offset: float,
                min_token_prob: float, alpha: float) -> SfxParams:
    thresholds = list(thresholds)
    caps = list(caps)
    if not 1 <= len(thresholds) <= MAX_CANDIDATES:
        raise ValueError(f"1..{MAX_CANDIDATES} support thresholds supported")
    if len(caps) > MAX_CANDIDATES:
        raise ValueError(f"at most {MAX_CANDIDATES} global caps supported")
    if max(thresholds) < 1:
        raise ValueError("support thresholds need a value >= 1")
    p = SfxParams()
    p.k = int(k)
    p.max_pattern_len = int(max_pattern_len)
    p.max_occurrences = int(max_occurrences)
    p.min_match_len = max(1, int(min_match_len))
    p.num_thresholds = len(thresholds)
    p.num_caps = len(caps)
    p.has_spec_factor = 0 if max_spec_factor is None else 1
    p.spec_factor = 0.0 if max_spec_factor is None else float(max_spec_factor)
    p.spec_offset = float(max_spec_offset)
    p.min_token_prob = float(min_token_prob)
    p.alpha = float(alpha)
    for i, t in enumerate(thresholds):
        p.thresholds[i] = max(-(2 ** 31), min(2 ** 31 - 1, int(t)))
    for i, c in enumerate(caps):
        p.caps[i] = max(-(2 ** 31), min(2 ** 31 - 1, int(c)))
    return p


def count_arg(t: torch.Tensor | None):
    """(tensor, is64) for an int32/int64 [B] count vector (None passes)."""
    if t is None:
        return None, 0
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    return t.contiguous(), int(t.dtype == torch.int64)


def make_batch(tokens: torch.Tensor, num_tokens: torch.Tensor,
               sampled: torch.Tensor | None = None,
               valid_count: torch.Tensor | None = None,
               mask: torch.Tensor | None = None, limit: int = 0):
    """SfxBatch plus the tensors it points to (keep them alive)."""
    if tokens.dtype != torch.int32 or not tokens.is_contiguous():
        raise ValueError("token_ids_gpu must be a contiguous int32 [B, S] "
                         "tensor (it is updated in place)")
    if tokens.dim() != 2 or tokens.shape[1] < 1:
        raise ValueError("token_ids_gpu must be [B, S] with S >= 1")
    b = tokens.shape[0]
    require_gpu(tokens, num_tokens, sampled, valid_count, mask)
    for name, t in (("num_tokens", num_tokens), ("sampled", sampled),
                    ("valid_count", valid_count), ("mask", mask)):
        if t is not None and (t.shape[0] != b or t.device != tokens.device):
            raise ValueError(f"{name} must have {b} rows on {tokens.device}")
    if sampled is not None and sampled.dim() != 2:
        raise ValueError("sampled_token_ids must be [B, T]")
    nt, nt64 = count_arg(num_tokens)
    vc, vc64 = count_arg(valid_count)
    keep = [tokens, nt, vc]
    bt = SfxBatch()
    bt.tokens = tokens.data_ptr()
    bt.batch = tokens.shape[0]
    bt.seq = tokens.shape[1]
    bt.num_tokens = nt.data_ptr()
    bt.num_tokens_is64 = nt64
    if sampled is not None:
        if sampled.dtype != torch.int32:
            sampled = sampled.to(torch.int32)
        sampled = sampled.contiguous()
        keep.append(sampled)
        bt.sampled = sampled.data_ptr()
        bt.num_sampled = sampled.shape[1]
    bt.valid_count = ptr(vc)
    bt.valid_count_is64 = vc64
    if mask is not None:
        mask = mask.to(torch.bool).contiguous()
        keep.append(mask)
        bt.mask = mask.data_ptr()
    bt.limit = int(limit)
    return bt, keep
