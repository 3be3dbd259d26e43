"""Host-only checks (no GPU): the C-ABI library loads and exports every
symbol include/locks_hip.h declares, rejects bad arguments before touching
the device, and the Python plugin surface mirrors the reference's."""
from __future__ import annotations

import ctypes
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "locks_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int32_t|int64_t)\s+(locks_\w+)\(",
                                 text, re.M)))


def test_library_exports_header_symbols():
    from locks import _lib
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.locks_abi_version() == _lib.ABI_VERSION


def _header_params():
    """name -> list of C parameter types, parsed from include/locks_hip.h."""
    text = open(os.path.join(ROOT, "include", "locks_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"(?:const char\*|int32_t|int64_t)\s+(locks_\w+)\(([^)]*)\);", text):
        params = [p.strip() for p in m.group(2).replace("\n", " ").split(",") if p.strip()]
        out[m.group(1)] = [] if params == ["void"] else params
    return out


def test_ctypes_signatures_match_the_header():
    """Every ctypes argtype list in locks/_lib.py has the header's parameter
    count and kind (pointer / int32 / int64 / float / double), and the return
    type matches: a drifted binding would pass arguments in the wrong slots."""
    from locks import _lib
    kinds = {"p": _lib._p, "i32": _lib._i32, "i64": _lib._i64, "f32": _lib._f32, "f64": _lib._f64}

    def kind(decl):
        if "*" in decl:
            return "p"
        t = decl.split()[0] if not decl.startswith("const ") else decl.split()[1]
        return {"int32_t": "i32", "int64_t": "i64", "float": "f32", "double": "f64"}[t]

    text = open(os.path.join(ROOT, "include", "locks_hip.h")).read()
    params = _header_params()
    assert set(params) == set(_lib.SIGNATURES)
    for name, decls in params.items():
        res, args = _lib.SIGNATURES[name]
        assert len(args) == len(decls), f"{name}: {len(args)} ctypes args, header has {len(decls)}"
        for i, (a, d) in enumerate(zip(args, decls)):
            assert a is kinds[kind(d)], f"{name} arg {i} ({d}): ctypes {a}"
        ret = re.search(r"(const char\*|int32_t|int64_t)\s+" + name + r"\(", text).group(1)
        want = {"int32_t": _lib._i32, "int64_t": _lib._i64}.get(ret)
        if want is not None:
            assert res is want, f"{name} returns {ret}"


def test_rejects_bad_geometry_without_device():
    from locks import _lib
    lib = _lib.load()
    args = [0, 0, 0] + [1] * 6 + [None] + [1, 1, 0, 1, 1, 1, 16, 1, 32, 1, 2, 4, 96, 16, 0.1, None]
    rc = lib.locks_score_rki4(*args)           # head_dim 96 is outside the contract
    assert rc == -1 and b"head_dim 96" in lib.locks_last_error()
    args[-4] = 64
    args[-3] = 128                             # page 128: outside the domain
    rc = lib.locks_score_rki4(*args)
    assert rc == -1 and b"page 128" in lib.locks_last_error()
    rc = lib.locks_decode_splitk(*([1, 8, 8] + [1, 8, 8, 8] * 2 + [1, 1, 8, 1, 1, 8, 8, 1, 1,
                                   8, 1, 1, 1, 1, 1, 2, 17, 128, 16, 4, 1, 0, 0.1, None]))
    assert rc == -1 and b"G=17" in lib.locks_last_error()
    # the DRAM-tier split: the tier struct is checked before any launch
    import ctypes
    targs = [1, 8, 8] + [1, 8, 8, 8] * 2 + [4, 1, 8, 1, 1, 8, 8, 1, 1, 8, 1, 1, 1, 1,
                                             1, 2, 4, 128, 16, 4, 1, 0, 0.1]
    assert lib.locks_decode_splitk_tier(*(targs + [None, None])) == -1
    assert b"null tier" in lib.locks_last_error()
    ts = _lib.TierSrc(hot_v=1, stage_v=1, pool_v=1, page2slot=1, vbo=1, stage_stride_block=8,
                      stage_stride_tok=8, stage_stride_head=8, num_blocks=3, hot_slots=2)
    assert lib.locks_decode_splitk_tier(*(targs + [ctypes.addressof(ts), None])) == -1
    assert b"num_blocks 3 != cache num_blocks 4" in lib.locks_last_error()
    ts.num_blocks, ts.k_tier = 4, 1
    assert lib.locks_decode_splitk_tier(*(targs + [ctypes.addressof(ts), None])) == -1
    assert b"k_tier needs" in lib.locks_last_error()
    ts.k_tier = 0
    # a tier laid out for another geometry, or a layer past the pool's layers
    for fields, msg in ((dict(n_kv=1, page=16, head_dim=128, num_layers=1), b"n_kv 1 / page 16"),
                        (dict(n_kv=2, page=32, head_dim=128, num_layers=1), b"page 32"),
                        (dict(n_kv=2, page=16, head_dim=64, num_layers=1), b"head_dim 64"),
                        (dict(n_kv=2, page=16, head_dim=128, num_layers=0), b"layer 0 outside")):
        for k, v in fields.items():
            setattr(ts, k, v)
        assert lib.locks_decode_splitk_tier(*(targs + [ctypes.addressof(ts), None])) == -1
        assert msg in lib.locks_last_error(), lib.locks_last_error()
    ts.num_layers, ts.layer = 2, 2
    assert lib.locks_decode_splitk_tier(*(targs + [ctypes.addressof(ts), None])) == -1
    assert b"layer 2 outside the pool's [0, 2)" in lib.locks_last_error()
    ts.layer, ts.stage_stride_tok = 1, 12
    assert lib.locks_decode_splitk_tier(*(targs + [ctypes.addressof(ts), None])) == -1
    assert b"staging strides" in lib.locks_last_error()
    assert lib.locks_host_device_pointer(None, None) == -1
    # two chunks (max_pages 4096) need the candidate workspace: rejected pre-launch
    rc = lib.locks_select_nrm_topb(*([1, 1, 1] + [1] * 7 + [0, 1, 2, 4, 1, 4096, 0, 0, None]))
    assert rc == -1 and b"workspace" in lib.locks_last_error()
    rc = lib.locks_derive_params(1, 1, 16, 0, 1, 0, 0.1, 1, 1, 1, None)
    assert rc == -1 and b"window" in lib.locks_last_error()


def test_workspace_and_chunk_math():
    from locks import _lib
    lib = _lib.load()
    c = lib.locks_score_auto_chunk(1, 2, 65536)
    assert c % 8 == 0 and 8 <= c <= 1024
    assert lib.locks_score_num_chunks(65536, c) == -(-65536 // c)
    assert lib.locks_select_workspace_bytes(1, 2, 65536) >= 2 * 65536 * 16
    assert lib.locks_select_workspace_bytes(0, 0, 1) == -1


def test_record_bytes_matches_reference_footprint():
    from locks.selection.rki4_state import record_bytes
    assert record_bytes(128, 16) == 834          # 818 B summary + 16 B tag
    assert record_bytes(128, 16, tagw=0) == 818


def test_config_surface(monkeypatch, tmp_path):
    from locks import LocksConfig
    c = LocksConfig()
    assert (c.variant, c.sink_pages, c.window_pages, c.quad_combine) == ("fast", 1, 1, "nrm")
    with pytest.raises(ValueError):
        LocksConfig(budget=1.5)
    with pytest.raises(ValueError):
        LocksConfig(quad_combine="sum")
    assert LocksConfig(variant="mem-kv").r8_screen is True
    monkeypatch.setenv("LOCKS_CONFIG", json.dumps({"budget_pages": 126}))
    monkeypatch.setenv("LOCKS_RKI4_Z", "64")
    c = LocksConfig.load({"sink_pages": 2})
    assert (c.budget_pages, c.sink_pages, c.rki4_zsplit) == (126, 2, 64)
    p = tmp_path / "c.yaml"
    p.write_text("budget: 0.05\n")
    monkeypatch.setenv("LOCKS_CONFIG", str(p))
    assert LocksConfig.load().budget == 0.05
    monkeypatch.setenv("LOCKS_CONFIG", json.dumps({"bogus": 1}))
    with pytest.raises(ValueError):
        LocksConfig.load()


def test_register_inert_then_registers_any_variant(monkeypatch, capsys):
    import locks
    from locks.backend import _runtime, register as regmod
    monkeypatch.delenv("LOCKS_CONFIG", raising=False)
    monkeypatch.setattr(regmod, "_APPLIED", False)
    locks.register()
    assert "INERT" in capsys.readouterr().out
    locks.register({"variant": "mem-v", "budget_pages": 126})   # the DRAM tier is served
    assert _runtime.get_config().variant == "mem-v"
    assert _runtime.get_config().budget_pages == 126


def test_register_refuses_vllm_without_backend_class(monkeypatch):
    """vLLM-ROCm importable but no vLLM backend class shipped: refuse at
    registration instead of patching the selector to a missing class."""
    import sys
    import types
    import locks
    from locks.backend import register as regmod
    fake_vllm = types.ModuleType("vllm")
    fake_platforms = types.ModuleType("vllm.platforms")
    fake_rocm = types.ModuleType("vllm.platforms.rocm")

    class RocmPlatform:
        @classmethod
        def get_attn_backend_cls(cls, *a, **k):
            return "vllm.v1.attention.backends.flash_attn.FlashAttentionBackend"

    fake_rocm.RocmPlatform = RocmPlatform
    fake_platforms.rocm = fake_rocm
    fake_vllm.platforms = fake_platforms
    monkeypatch.setitem(sys.modules, "vllm", fake_vllm)
    monkeypatch.setitem(sys.modules, "vllm.platforms", fake_platforms)
    monkeypatch.setitem(sys.modules, "vllm.platforms.rocm", fake_rocm)
    monkeypatch.setattr(regmod, "_APPLIED", False)
    with pytest.raises(NotImplementedError, match="LocksEngine"):
        locks.register({"budget_pages": 126})
    assert RocmPlatform.get_attn_backend_cls().endswith("FlashAttentionBackend")   # untouched


def test_geometry_contract():
    from locks.selection import Rki4State
    for d in (64, 128, 256):
        for page in (16, 32, 64):
            Rki4State.validate_geometry(head_dim=d, G=16, page=page)
    for kw in (dict(head_dim=96, G=4, page=16), dict(head_dim=128, G=17, page=16),
               dict(head_dim=128, G=4, page=128), dict(head_dim=512, G=4, page=16),
               dict(head_dim=128, G=4, page=8)):
        with pytest.raises(AssertionError):
            Rki4State.validate_geometry(**kw)


def test_product_path_has_no_oracle_import():
    """Nothing under the shipped package imports the oracle or numpy CPU math."""
    pkg = os.path.join(ROOT, "locks-kv_amd", "locks")
    for dp, _, fs in os.walk(pkg):
        for f in fs:
            if f.endswith(".py"):
                src = open(os.path.join(dp, f)).read()
                assert "oracle" not in src.replace("no CPU or PyTorch fallback", ""), f


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from locks import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "_LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.LocksLibraryError):
        _lib.load()


def test_mla_entries_reject_bad_geometry_without_device():
    from locks import _lib
    lib = _lib.load()
    # locks_mla_score: kv_lora_rank 256 is outside this build
    args = [1, 16 * 576, 576] + [1] * 9 + [16 * 576, 576, 8, 1, 64, 64, 1, 1, 64, 64, 64, 1, 16,
                                             256, 64, 16, 0.1, None]
    assert lib.locks_mla_score(*args) == -1 and b"geometry" in lib.locks_last_error()
    args[24] = 17                                       # 17 heads
    args[25] = 512
    assert lib.locks_mla_score(*args) == -1 and b"n_heads=17" in lib.locks_last_error()
    args[24] = 16
    args[22] = 3                                        # odd chunk
    assert lib.locks_mla_score(*args) == -1 and b"chunk 3" in lib.locks_last_error()
    args[22] = 64
    args[10] = None                                     # rk8 without rks
    assert lib.locks_mla_score(*args) == -1 and b"rk8 and rks" in lib.locks_last_error()
    # the int8 RoPE builder: strides must allow 16-byte loads
    assert lib.locks_mla_build_rope(1, 16 * 576 + 4, 576, 8, 1, 1, None, 1, 1, None) == -1
    assert b"multiples of 8" in lib.locks_last_error()
    # decode: split above the partial buffers' bound
    dargs = [1, 16 * 576, 576, 1, 16 * 576, 576, 8, 1, 64, 64, 1, 64, 64, 1, 1, 1, 1, 1,
             1, 16, 512, 64, 16, 513, 4, 0.1, None]
    assert lib.locks_mla_decode_splitk(*dargs) == -1 and b"split=513" in lib.locks_last_error()
    margs = [1, 1, 1, 1, 64, 1, 16 * 512, 510, 0, None, 16, 1, 16, 512, 8, 4, None]
    assert lib.locks_mla_decode_merge(*margs) == -1 and b"multiples of 4" in lib.locks_last_error()
    assert 2 <= lib.locks_mla_score_auto_chunk(1, 8192) <= 1024
    assert lib.locks_mla_score_auto_chunk(1, 8192) % 2 == 0
    # the build takes d = 512 (the latent) only at page 16, and no d = 96
    bargs = [1, 16 * 576, 576, 0, 8, 1, 1, 1, 96, 16] + [1] * 6 + [None, 1, None]
    assert lib.locks_build_rki4(*bargs) == -1 and b"d=96" in lib.locks_last_error()
    bargs[8:10] = [512, 32]
    assert lib.locks_build_rki4(*bargs) == -1 and b"d=512 page=32" in lib.locks_last_error()



def test_refresh_entries_reject_bad_arguments_without_device():
    from locks import _lib
    lib = _lib.load()
    # locks_refresh_blocks(mode, bt, bt_stride, sl, n_req, rows, n_rows, max_fin, page, num_blocks,
    #                      k_layers, n_layers, k_sb, k_st, k_sh, n_kv, tag, tag_blocks, mark,
    #                      blocks, count, stream)
    ok = [1, 1, 64, 1, 2, None, 0, 8, 16, 100, None, 0, 0, 0, 0, 1, None, 100, 1, 1, 1, None]
    a = list(ok); a[0] = 7
    assert lib.locks_refresh_blocks(*a) == -1 and b"unknown mode 7" in lib.locks_last_error()
    a = list(ok); a[7] = 65                              # max_fin past the block-table width
    assert lib.locks_refresh_blocks(*a) == -1 and b"max_fin 65" in lib.locks_last_error()
    a = list(ok); a[0] = 2                               # delta needs K pointers and the tag slab
    assert lib.locks_refresh_blocks(*a) == -1 and b"delta needs" in lib.locks_last_error()
    a = list(ok); a[18] = None
    assert lib.locks_refresh_blocks(*a) == -1 and b"null pointer" in lib.locks_last_error()
    # locks_build_rki4_layers: geometry and the slab-blocks bound
    bl = [1, 2, 16 * 8 * 128, 8 * 128, 128, 100, 1, None, 4, 8, 128, 16, 100] + [1] * 6 + [None, 1, None]
    b = list(bl); b[10] = 96
    assert lib.locks_build_rki4_layers(*b) == -1 and b"d=96" in lib.locks_last_error()
    b = list(bl); b[11] = 8                              # page 8: outside the domain
    assert lib.locks_build_rki4_layers(*b) == -1 and b"page=8" in lib.locks_last_error()
    b = list(bl); b[12] = 50                             # slab smaller than the K pool bound
    assert lib.locks_build_rki4_layers(*b) == -1 and b"bad geometry" in lib.locks_last_error()
    b = list(bl); b[3] = 12                              # token stride not a multiple of 8
    assert lib.locks_build_rki4_layers(*b) == -1 and b"multiples of 8" in lib.locks_last_error()
    assert lib.locks_calib_read(None, 64, None, None) == -1


def test_engine_and_producers_validate_on_the_host():
    import torch
    from types import SimpleNamespace
    from locks.backend.engine import LocksEngine
    from locks.config import LocksConfig
    from locks.selection import rki4_build_tail
    with pytest.raises(ValueError):                      # summary records in the engine page
        LocksEngine(LocksConfig(variant="mem-kv", mem_summary_cache=True), [torch.zeros(1)],
                    num_heads_q=8, num_heads_kv=2, head_dim=128, block_size=16, max_num_seqs=1,
                    max_model_len=64)
    with pytest.raises(ValueError):
        LocksEngine(LocksConfig(), [torch.zeros(1)], num_heads_q=6, num_heads_kv=4,
                    head_dim=128, block_size=16, max_num_seqs=1, max_model_len=64)
    with pytest.raises(ValueError):
        LocksEngine(LocksConfig(), [], num_heads_q=8, num_heads_kv=2, head_dim=128,
                    block_size=16, max_num_seqs=1, max_model_len=64)
    st = SimpleNamespace(L=2, NB=4)
    K = torch.zeros(4, 16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):                      # one K view for a 2-layer state
        rki4_build_tail(st, [K], torch.zeros(1, 4, dtype=torch.int32),
                        torch.ones(1, dtype=torch.int32), 1)
    with pytest.raises(TypeError):                       # layers of different strides
        rki4_build_tail(st, [K, K.transpose(1, 2).contiguous().transpose(1, 2)],
                        torch.zeros(1, 4, dtype=torch.int32), torch.ones(1, dtype=torch.int32), 1)
