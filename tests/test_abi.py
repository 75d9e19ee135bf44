"""The C ABI without a GPU: the library loads, exports every function the
header declares, reports the header's ABI version, and the ctypes mirrors
of the header structs have the C layout (checked against gcc's sizeof /
offsetof of the header itself).  No kernel is launched."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from suffixgpu_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "suffixgpu_amd.h"
ROCM_INCLUDE = Path("/opt/rocm/include")


def header_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sfx_\w+)\s*\(", text)))


def header_define(name: str) -> int:
    m = re.search(rf"#define\s+{name}\s+\(?(-?\d+)\)?", HEADER.read_text())
    assert m, name
    return int(m.group(1))


@pytest.fixture(scope="module")
def so():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} missing: run `python -m "
                    "suffixgpu_amd.build` first")
    return ctypes.CDLL(str(_lib.LIB_PATH))


def test_header_declares_the_reference_operator_set():
    fns = header_functions()
    for name in ("sfx_scatter_append", "sfx_match_back",
                 "sfx_first_occurrences", "sfx_sa_search", "sfx_expand_chain",
                 "sfx_local_gather", "sfx_local_forward", "sfx_global_query",
                 "sfx_propose_step", "sfx_sa_build", "sfx_sa_keys",
                 "sfx_index_swap"):
        assert name in fns


def test_library_exports_every_declared_function(so):
    missing = [f for f in header_functions() if not hasattr(so, f)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_abi_version_and_constants(so):
    so.sfx_abi_version.restype = ctypes.c_int32
    assert so.sfx_abi_version() == header_define("SFX_ABI_VERSION")
    assert _lib.ABI_VERSION == header_define("SFX_ABI_VERSION")
    assert _lib.MAX_CANDIDATES == header_define("SFX_MAX_CANDIDATES")
    assert _lib.EINVAL == header_define("SFX_EINVAL")
    assert _lib.ENOSCRATCH == header_define("SFX_ENOSCRATCH")
    assert (_lib.NOALLOC_SCRATCH_BYTES
            == header_define("SFX_NOALLOC_SCRATCH_BYTES"))
    so.sfx_sa_group_cap.restype = ctypes.c_int32
    assert so.sfx_sa_group_cap() == 2048  # the value the header documents
    assert _lib.NOALLOC_MAX_ROWS == header_define("SFX_NOALLOC_MAX_ROWS")
    assert _lib.SA_ROUNDS_RADIX == header_define("SFX_SA_ROUNDS_RADIX")
    assert (_lib.SA_ROUNDS_EXPECT_FINAL
            == header_define("SFX_SA_ROUNDS_EXPECT_FINAL"))


def test_workspace_sizes_are_host_only(so):
    lib = _lib.lib()
    p = _lib.make_params(16, 32, 128, 1, [1, 2, 4, 8, 16, 32, 64, 128],
                         [32, 16, 8, 4, 2], 2.0, 0.0, 0.1, 0.0)
    assert lib.sfx_step_workspace_size(p, 64, 1 << 16) > 0
    assert lib.sfx_global_query_workspace_size(p, 64, 1 << 16) > 0
    assert lib.sfx_sa_build_workspace_size(1 << 22) >= 40 * (1 << 22)
    assert lib.sfx_sa_build_workspace_size(-1) == 0


def test_argument_errors_are_reported_before_any_launch():
    lib = _lib.lib()
    # invalid sizes are rejected on the host: nothing is enqueued
    assert lib.sfx_sa_keys(None, None, 16, 16, 3, None, None, None) == -1
    assert lib.sfx_sa_keys(None, None, 16, 17, 32, None, None, None) == -1
    assert lib.sfx_sa_keys(None, None, 16, 0, 32, None, None, None) == 0
    # first4 must be 16-byte aligned (checked before any launch)
    assert lib.sfx_sa_keys(None, None, 16, 0, 32, None, 8, None) == -1
    assert lib.sfx_sa_build(None, -1, 0, None, 0, None, 0, None) == -1
    # sfx_sa_build_rounds takes two flag bits; m = 1 needs no workspace,
    # so only the flags can be wrong (a valid call enqueues nothing)
    assert lib.sfx_sa_build_rounds(1, 1, 1, 4, None, 0, None) == -1
    assert lib.sfx_sa_build_rounds(1, 1, 1, -1, None, 0, None) == -1
    assert lib.sfx_sa_build_rounds(1, 1, 1, 3, None, 0, None) == 0
    assert lib.sfx_index_swap(None, None, None, None, -1, None, 0,
                              None) == -1
    assert lib.sfx_index_swap(None, None, None, None, 16, None, 0,
                              None) == -1
    # a document that would end past the delta (its SEP at capacity)
    docs = (_lib.SfxAppendDoc * 2)(_lib.SfxAppendDoc(1, 10, 0),
                                   _lib.SfxAppendDoc(1, 10, 6))
    assert lib.sfx_delta_append(docs, 2, 1, 16, None, 17, None) == -1
    assert lib.sfx_delta_append(docs, 2, 1, 17, None, 18, None) == -1
    assert lib.sfx_delta_append(docs, -1, 1, 17, None, 0, None) == -1
    assert lib.sfx_delta_shift(1, 16, 8, 9, None, None) == -1
    assert lib.sfx_delta_shift(None, 16, 1, 1, None, None) == -1
    # key rows must be 16-byte aligned (they are read as 16-byte words).
    # An empty batch with a stand-in workspace runs every host check and
    # launches nothing, so the addresses are never dereferenced.
    p = _lib.make_params(4, 8, 16, 1, [1], [8, 4, 2], None, 0.0, 0.0, 0.0)
    out = _lib.SfxGlobalOut()
    for key, rc in ((0x100008, -1), (0x100010, 0)):
        ix = _lib.SfxIndex(0x200000, 0x300000, 1 << 10, 0x400000, 1 << 10,
                           0x500000, key, 32)
        assert lib.sfx_global_query(ctypes.byref(p), ctypes.byref(ix), None,
                                    0, 1, None, ctypes.byref(out), 0x600000,
                                    1 << 40, None) == rc
    # a key-row selector needs the first buffer; the second may be NULL
    # (none while the selector is set) and is 16-byte aligned otherwise
    for alt, rc in ((0, 0), (0x700008, -1), (0x700010, 0)):
        ix = _lib.SfxIndex(0x200000, 0x300000, 1 << 10, 0x400000, 1 << 10,
                           0x500000, 0x100010, 32, alt, 0x800000)
        assert lib.sfx_global_query(ctypes.byref(p), ctypes.byref(ix), None,
                                    0, 1, None, ctypes.byref(out), 0x600000,
                                    1 << 40, None) == rc


def test_noalloc_step_rejects_batches_beyond_the_scratch():
    """sfx_propose_step_noalloc checks on the host, before it touches the
    device, that the batch fits the static scratch: more rows than its
    counter arrays hold, or a workspace larger than the array.  Stand-in
    addresses, so this runs only where no GPU is visible."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("host-only check with stand-in addresses")
    lib = _lib.lib()
    p = _lib.make_params(16, 32, 128, 1, [1, 2, 4, 8, 16, 32, 64, 128],
                         [32, 16, 8, 4, 2], 2.0, 0.0, 0.1, 0.0)
    for b, dcap in ((_lib.NOALLOC_MAX_ROWS + 1, 1 << 12), (600, 1 << 22)):
        ix = _lib.SfxIndex(0x200000, 0x300000, 1 << 12, 0x400000, dcap,
                           0x500000, None, 0, None, None, None, None, 0)
        bt = _lib.SfxBatch()
        bt.tokens = 0x100000
        bt.batch = b
        bt.seq = 64
        bt.num_tokens = 0x200000
        bt.sampled = 0x300000
        bt.num_sampled = 17
        bt.limit = 64
        rc = lib.sfx_propose_step_noalloc(ctypes.byref(p), ctypes.byref(ix),
                                          ctypes.byref(bt), 0x400000,
                                          0x500000, 0x600000, None)
        assert rc == _lib.ENOSCRATCH, (b, dcap, rc)
    with pytest.raises(_lib.SuffixGPUError, match="static step scratch"):
        _lib.check(_lib.ENOSCRATCH, "step")


def test_ingest_entry_points_check_arguments_on_the_host():
    """Device-side ingest rejects bad geometry before any launch."""
    lib = _lib.lib()
    lay = (ctypes.c_int64 * 8)()
    assert lib.sfx_ingest_layout(0, 16, lay) == -1
    assert lib.sfx_ingest_layout(1 << 10, 1 << 8, lay) == 0
    # unaligned state, too many documents, missing progress table
    args = (0x100100, 0x200000, 1 << 10, 0x300000, 1 << 8, 0x400000,
            0x500000, 0x600000, 4, 8, 0x700000, 0, 0x800000, 0)
    assert lib.sfx_ingest_docs(0x100104, *args[1:], 4, 100, None) == -1
    assert lib.sfx_ingest_docs(*args, _lib.INGEST_MAX_DOCS + 1, 100,
                               None) == -1
    assert lib.sfx_ingest_active(*args, 4, None, 16, 0, 64, 48, 100,
                                 None) == -1
    assert lib.sfx_ingest_active(*args, 4, 0x900000, 0, 0, 64, 48, 100,
                                 None) == -1
    # more documents than rows of the token buffer
    assert lib.sfx_ingest_active(*args, 5, 0x900000, 16, 0, 64, 48, 100,
                                 None) == -1


STRUCT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "suffixgpu_amd.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f))
#define S(T) printf(#T " %zu\n", sizeof(T))
int main(void) {
  S(sfx_params); F(sfx_params, k); F(sfx_params, spec_factor);
  F(sfx_params, alpha); F(sfx_params, thresholds); F(sfx_params, caps);
  S(sfx_index); F(sfx_index, delta_len); F(sfx_index, sa_key);
  F(sfx_index, key_width); F(sfx_index, sa_key_alt);
  F(sfx_index, key_select); F(sfx_index, gram_slots);
  F(sfx_index, delta_entries); F(sfx_index, delta_buckets);
  S(sfx_batch); F(sfx_batch, num_tokens_is64); F(sfx_batch, sampled);
  F(sfx_batch, valid_count_is64); F(sfx_batch, mask); F(sfx_batch, limit);
  S(sfx_global_out); F(sfx_global_out, draft_score);
  S(sfx_append_doc); F(sfx_append_doc, n); F(sfx_append_doc, dst);
  printf("SFX_APPEND_MAX_DOCS %d\n", SFX_APPEND_MAX_DOCS);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None
                    or not (ROCM_INCLUDE / "hip").is_dir(),
                    reason="needs gcc and the ROCm headers")
def test_struct_layouts_match_the_header(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(STRUCT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}",
                    f"-I{ROCM_INCLUDE}", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True,
                         text=True).stdout
    c = dict(line.rsplit(" ", 1) for line in out.strip().splitlines())
    mirrors = {"sfx_params": _lib.SfxParams, "sfx_index": _lib.SfxIndex,
               "sfx_batch": _lib.SfxBatch, "sfx_global_out": _lib.SfxGlobalOut,
               "sfx_append_doc": _lib.SfxAppendDoc}
    assert int(c.pop("SFX_APPEND_MAX_DOCS")) == _lib.APPEND_MAX_DOCS
    for key, val in c.items():
        if "." in key:
            t, f = key.split(".")
            assert getattr(mirrors[t], f).offset == int(val), key
        else:
            assert ctypes.sizeof(mirrors[key]) == int(val), key


def test_delta_index_build_checks_arguments_on_the_host():
    """sfx_delta_index_build rejects a bucket count that is not a power of
    two in 2^10 .. 2^17, a missing buffer, misaligned entries, a
    misaligned or short workspace, and a capacity out of range, before any
    launch."""
    lib = _lib.lib()
    d = 1 << 12
    need = lib.sfx_delta_index_bytes(d)
    assert need > 0 and lib.sfx_delta_index_bytes(0) == 0
    ok = (0x100000, 0x200000, d, 0x300000, 0x400000)
    assert lib.sfx_delta_index_build(0x100000, 0x200000, d, 0x300008,
                                     0x400000, 1 << 10, 0x500000, need,
                                     None) == -1  # entries 16-byte aligned
    for buckets in (1 << 9, 3 << 10, 1 << 18):
        assert lib.sfx_delta_index_build(*ok, buckets, 0x500000, need,
                                          None) == -1
    assert lib.sfx_delta_index_build(*ok, 1 << 10, 0x500010, need,
                                      None) == -1
    assert lib.sfx_delta_index_build(*ok, 1 << 10, 0x500000, need - 1,
                                     None) == -1
    assert lib.sfx_delta_index_build(None, *ok[1:], 1 << 10, 0x500000, need,
                                     None) == -1
    assert lib.sfx_delta_index_build(0x100000, 0x200000, 0, 0x300000,
                                     0x400000, 1 << 10, 0x500000, need,
                                     None) == -1
