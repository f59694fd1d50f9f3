"""The C ABI without a GPU: the library loads, exports every entry point include/nvs_amd.h declares, and rejects
bad arguments on the host before any launch. CPU only (no call here reaches a kernel)."""
import ctypes
import pathlib
import re

import pytest

from nvs_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "nvs_amd.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(nvs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version_and_empty_error(lib):
    assert lib.nvs_abi_version() == _lib.ABI_VERSION == 9
    assert isinstance(lib.nvs_last_error(), bytes)


def test_argument_counts_match_the_header(lib):
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, argtypes in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))


def attn_args(**over):
    args = dict(q=1 << 20, q_ts=4096, q_hs=128, n_tokens=8, k=1 << 21, v=1 << 22, cache_blocks=4, c_bs=262144,
                c_ts=1024, c_hs=128, bt=1 << 23, bt_rs=4, bt_width=4, cu_q=1 << 24, cu_k=1 << 25, ctx=None,
                qlen=0, rows=1, mq=8, mk=1024, h=32, hkv=8, d=128, bs=256, scale=0.088, causal=1,
                dtype=_lib.DTYPE_BF16, out=1 << 26, o_ts=4096, o_hs=128, counters=None, ws=None, ws_bytes=0,
                stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over, status", [
    (dict(d=96), _lib.NVS_ERR_UNSUPPORTED),
    (dict(dtype=_lib.DTYPE_F32), _lib.NVS_ERR_UNSUPPORTED),
    (dict(h=30), _lib.NVS_ERR_INVALID),
    (dict(bs=48), _lib.NVS_ERR_UNSUPPORTED),
    (dict(q=(1 << 20) + 2), _lib.NVS_ERR_INVALID),
    (dict(c_ts=1020), _lib.NVS_ERR_INVALID),
    (dict(cu_k=None), _lib.NVS_ERR_INVALID),
    (dict(cu_q=None, cu_k=None, ctx=None), _lib.NVS_ERR_INVALID),
    (dict(scale=0.0), _lib.NVS_ERR_INVALID),
    (dict(bt_width=0), _lib.NVS_ERR_INVALID),
    (dict(rows=1, mk=4096), _lib.NVS_ERR_WORKSPACE),   # one row: the plan splits its keys, partials needed
    (dict(rows=1, mk=4096, ws=1 << 27, ws_bytes=1 << 30), _lib.NVS_ERR_INVALID),   # and the merge's counters
])
def test_attention_rejects_bad_arguments_without_launching(lib, over, status):
    assert lib.nvs_paged_attention(*attn_args(**over)) == status
    assert lib.nvs_last_error()


def test_attention_workspace_plan(lib):
    n = ctypes.c_size_t()
    # batch 64 x 8 kv heads fills one resident round: unsplit, no partials
    assert lib.nvs_paged_attention_workspace_size(64, 32, 8, 128, 8, 4096, ctypes.byref(n)) == 0
    assert n.value == 0
    # batch 2: the keys are split to fill the chip, partials need a workspace
    assert lib.nvs_paged_attention_workspace_size(2, 32, 8, 128, 8, 4096, ctypes.byref(n)) == 0
    assert n.value > 0
    # batch 32 (256 units, one per CU) stays unsplit; batch 16 (128 units) is split
    assert lib.nvs_paged_attention_workspace_size(32, 32, 8, 128, 8, 4096, ctypes.byref(n)) == 0
    assert n.value == 0
    assert lib.nvs_paged_attention_workspace_size(16, 32, 8, 128, 8, 4096, ctypes.byref(n)) == 0
    assert n.value > 0
    # at most 64 splits per unit whatever max_seqlen_k: partials of 32 rows x (128 + 2) fp32 per split
    assert lib.nvs_paged_attention_workspace_size(1, 32, 8, 128, 8, 1 << 17, ctypes.byref(n)) == 0
    assert 0 < n.value <= 8 * 64 * 32 * 130 * 4 + 256
    small = ctypes.c_size_t()
    assert lib.nvs_paged_attention_workspace_size(1, 32, 8, 128, 8, 64, ctypes.byref(small)) == 0
    assert small.value == 0            # 64 keys: one split, no partials
    assert lib.nvs_paged_attention_workspace_size(1, 32, 8, 64, 8, 64, ctypes.byref(small)) == _lib.NVS_ERR_UNSUPPORTED


def test_sampler_rejects_bad_arguments_without_launching(lib):
    n = ctypes.c_size_t()
    # any top-k window is served (windows past 1024 values take the exact path); a negative one is invalid
    assert lib.nvs_spec_accept_workspace_size(64, 7, 512, 151936, 2000, ctypes.byref(n)) == 0
    assert lib.nvs_spec_accept_workspace_size(64, 7, 512, 151936, -1, ctypes.byref(n)) == _lib.NVS_ERR_INVALID
    assert lib.nvs_spec_accept_workspace_size(64, 7, 512, 151936, 64, ctypes.byref(n)) == 0
    assert n.value == 512 * 32              # a 32-byte record per position
    # fixed-length call whose position count is not B*(k+1)
    st = lib.nvs_spec_accept(1 << 20, _lib.DTYPE_F32, 100, 1 << 20, 1 << 20, 1 << 20, 64, 0, 1 << 20, 1 << 20, None,
                             1 << 20, 1 << 20, 4, 7, 31, 100, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1024, None)
    assert st == _lib.NVS_ERR_INVALID
    # workspace too small
    st = lib.nvs_spec_accept(1 << 20, _lib.DTYPE_F32, 100, 1 << 20, 1 << 20, 1 << 20, 64, 0, 1 << 20, 1 << 20, None,
                             1 << 20, 1 << 20, 4, 7, 32, 100, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 16, None)
    assert st == _lib.NVS_ERR_WORKSPACE
    assert lib.nvs_probs_from_logits(1 << 20, 9, 100, 4, 100, 1, 1 << 20, None, None, 0, 0, 1 << 20, None, 0,
                                     None) == _lib.NVS_ERR_INVALID
    assert lib.nvs_race(1 << 20, 10, 1 << 20, 10, 3, 100, 1 << 20, 1 << 20, None, 0, None) == _lib.NVS_ERR_INVALID
    # the one-launch race needs its zeroed row counters
    assert lib.nvs_race(1 << 20, 100, 1 << 20, 100, 3, 100, 1 << 20, None, 1 << 20, 1 << 20,
                        None) == _lib.NVS_ERR_INVALID
    assert lib.nvs_accept_random(1 << 20, 1 << 20, 1 << 20, None, 1 << 20, 1 << 20, 2, 3, 8, 100, 1 << 20, 1 << 20,
                                 None, 1 << 20, 1 << 20, None) == _lib.NVS_ERR_INVALID


def test_store_kvcache_rejects_bad_arguments(lib):
    nhd = (100, 256, 256 * 1024, 1024, 128)   # blocks, block size, block / token / head strides
    assert lib.nvs_store_kvcache(1 << 20, 1024, 1 << 20, 1024, 1 << 21, 1 << 22, *nhd, 1 << 23, 4, 8, 128, 7,
                                 None) == _lib.NVS_ERR_INVALID        # unknown dtype
    assert lib.nvs_store_kvcache(1 << 20, 512, 1 << 20, 1024, 1 << 21, 1 << 22, *nhd, 1 << 23, 4, 8, 128,
                                 _lib.DTYPE_BF16, None) == _lib.NVS_ERR_INVALID   # key rows shorter than 8 x 128
    assert lib.nvs_store_kvcache(1 << 20, 1024, 1 << 20, 1024, 1 << 21, 1 << 22, 100, 0, 1, 1, 1, 1 << 23, 4, 8,
                                 128, _lib.DTYPE_BF16, None) == _lib.NVS_ERR_INVALID   # block size 0
    assert lib.nvs_store_kvcache(1 << 20, 1024, 1 << 20, 1024, 1 << 21, 1 << 22, 100, 256, -1, 1024, 128, 1 << 23,
                                 4, 8, 128, _lib.DTYPE_BF16, None) == _lib.NVS_ERR_INVALID   # negative stride
    assert lib.nvs_store_kvcache(None, 0, None, 0, None, None, 0, 256, 0, 0, 0, None, 0, 8, 128, _lib.DTYPE_BF16,
                                 None) == 0


def test_qk_norm_rope_store_rejects_bad_arguments(lib):
    def call(**over):
        a = dict(q=1 << 20, q_ts=6144, k=1 << 21, k_ts=6144, v=1 << 22, v_ts=6144, pos=1 << 23, qw=None, kw=None,
                 eps=1e-6, cs=1 << 24, n_cs=4096, slots=None, kc=None, vc=None, blocks=0, block_size=256,
                 bs=256 * 1024, ts=1024, hs=128, qo=1 << 25,
                 qo_ts=4096, ko=None, ko_ts=0, T=4, hq=32, hkv=8, d=128, dtype=_lib.DTYPE_BF16, stream=None)
        a.update(over)
        return lib.nvs_qk_norm_rope_store(*a.values())
    assert call(dtype=_lib.DTYPE_F32) == _lib.NVS_ERR_UNSUPPORTED
    assert call(d=64) == _lib.NVS_ERR_UNSUPPORTED
    assert call(q=None) == _lib.NVS_ERR_INVALID            # query heads without q
    assert call(k_ts=512) == _lib.NVS_ERR_INVALID          # shorter than 8 heads x 128
    assert call(slots=1 << 26) == _lib.NVS_ERR_INVALID     # slots without caches
    assert call(slots=1 << 26, kc=1 << 27, vc=1 << 28, blocks=4, block_size=0) == _lib.NVS_ERR_INVALID
    assert call(slots=1 << 26, kc=1 << 27, vc=1 << 28, blocks=4, hs=-128) == _lib.NVS_ERR_INVALID
    assert call(n_cs=0) == _lib.NVS_ERR_INVALID
    assert call(T=0) == _lib.NVS_OK                        # nothing to do, nothing launched


def test_rms_norm_and_silu_mul_reject_bad_arguments(lib):
    def norm(**over):
        a = dict(x=1 << 20, x_rs=4096, res=None, res_rs=0, w=1 << 21, eps=1e-6, out=1 << 22, out_rs=4096, rows=4,
                 hidden=4096, dtype=_lib.DTYPE_BF16, stream=None)
        a.update(over)
        return lib.nvs_rms_norm(*a.values())
    assert norm(dtype=_lib.DTYPE_F32) == _lib.NVS_ERR_UNSUPPORTED
    assert norm(hidden=4100) == _lib.NVS_ERR_UNSUPPORTED      # not a multiple of 8
    assert norm(hidden=16384, x_rs=16384, out_rs=16384) == _lib.NVS_ERR_UNSUPPORTED   # above 8192
    assert norm(x_rs=2048) == _lib.NVS_ERR_INVALID            # shorter than the row
    assert norm(res=1 << 23, res_rs=1000) == _lib.NVS_ERR_INVALID
    assert norm(x=(1 << 20) + 2) == _lib.NVS_ERR_UNSUPPORTED  # not 16-byte aligned
    assert norm(w=None) == _lib.NVS_ERR_INVALID
    assert norm(rows=0) == _lib.NVS_OK                        # nothing to do, nothing launched

    def silu(**over):
        a = dict(x=1 << 20, x_rs=24576, out=1 << 22, out_rs=12288, rows=4, width=12288, dtype=_lib.DTYPE_BF16,
                 stream=None)
        a.update(over)
        return lib.nvs_silu_and_mul(*a.values())
    assert silu(dtype=_lib.DTYPE_F32) == _lib.NVS_ERR_UNSUPPORTED
    assert silu(width=12) == _lib.NVS_ERR_UNSUPPORTED
    assert silu(x_rs=12288) == _lib.NVS_ERR_INVALID           # holds the gate only
    assert silu(out=None) == _lib.NVS_ERR_INVALID
    assert silu(rows=0) == _lib.NVS_OK
