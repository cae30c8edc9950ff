"""CPU checks of the C ABI: the library loads, exports every symbol declared in
include/fsi.h, and rejects bad arguments with the documented status codes
before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "fsi.h").read_text()
    return sorted(set(re.findall(r"FSI_API[^;(]*?\b(fsi_\w+)\s*\(", text, flags=re.S)))


def test_header_declares_symbols():
    syms = _declared_symbols()
    assert "fsi_pattention_fwd" in syms and len(syms) >= 5


def test_library_exports_every_declared_symbol(fsi):
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    for name in _declared_symbols():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes signature table"
    assert set(_lib.SIGNATURES) == set(_declared_symbols())
    assert L.fsi_abi_version() == 1


def test_status_strings(fsi):
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    assert L.fsi_status_string(0) == b"ok"
    assert L.fsi_status_string(-3) == b"index out of range"


def _patt(L, **over):
    # Fake but aligned addresses: every case below must be rejected by host-side
    # validation, which runs before any HIP call (these tests also run on GPU boxes).
    a = dict(x=4096, ldx=64, kg=8192, ku=12288, ldk=64, v=16384, ldv=64, act_ptr=None, n_active=0, block_n=64, M=4,
             K=64, N_p=128, D_out=64, dtype=1, activation=0, rounding=1, out=20480, ldo=64, ws=24576, ws_bytes=16,
             err=None, stream=None)
    a.update(over)
    return L.fsi_pattention_fwd(a["x"], a["ldx"], a["kg"], a["ku"], a["ldk"], a["v"], a["ldv"], a.get("vt", 0), a["act_ptr"],
                                a["n_active"], a["block_n"], a["M"], a["K"], a["N_p"], a["D_out"], a["dtype"],
                                a["activation"], a["rounding"], a["out"], a["ldo"], a["ws"], a["ws_bytes"], a["err"],
                                a["stream"])


def test_pattention_argument_errors(fsi):
    """Validation happens on the host and returns before any HIP call."""
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    assert _patt(L, dtype=7) == _lib.FSI_ERR_DTYPE
    assert _patt(L, activation=9) == _lib.FSI_ERR_INVALID_ARG
    assert _patt(L, rounding=5) == _lib.FSI_ERR_INVALID_ARG
    assert _patt(L, block_n=48) == _lib.FSI_ERR_SHAPE
    assert _patt(L, ku=None) == _lib.FSI_ERR_INVALID_ARG            # swiglu needs k_up
    assert _patt(L, K=60, ldx=60, ldk=60) == _lib.FSI_ERR_ALIGN      # bf16 K % 8
    assert _patt(L, ldx=32) == _lib.FSI_ERR_SHAPE                    # ld < K
    assert _patt(L, n_active=3) == _lib.FSI_ERR_INVALID_ARG          # list length without list
    assert _patt(L) == _lib.FSI_ERR_WORKSPACE                         # 16-byte workspace
    assert _patt(L, x=None) == _lib.FSI_ERR_INVALID_ARG
    assert b"null" in L.fsi_last_error()
    assert _patt(L, dtype=7) == _lib.FSI_ERR_DTYPE
    assert b"dtype" in L.fsi_last_error()


def test_workspace_sizes_are_consistent(fsi):
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    a = L.fsi_pattention_workspace_size(64, 4096, 4096, 4096, 1)
    b = L.fsi_pattention_workspace_size(64, 4096, 4096, 4096 * 2, 1)
    assert 0 < a < b
    assert L.fsi_pattention_workspace_size(64, 512, 512, 512, 0) >= 64 * 512 * 4


def test_python_ops_refuse_cpu_tensors(fsi):
    import torch

    x = torch.randn(4, 64).bfloat16()
    w = torch.randn(128, 64).bfloat16()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fsi.triton_pattention(x, w, w, k_up=w)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fsi.triton_fused_swiglu(x, x)


def test_module_matches_reference_interface(fsi):
    import torch

    m = fsi.FovealPattentionMLP(hidden_dim=128, intermediate_dim=512, base_blocks=2, remote_blocks=3,
                                dtype=torch.float32)
    names = set(dict(m.named_parameters()))
    assert names == {"k_gate", "k_up", "v", "q_proj_16d.weight", "block_keys_16d", "out_proj_16d.weight"}
    assert "offsets" in dict(m.named_buffers())
    assert m.num_blocks == 8 and m.total_active_blocks == 5
    with pytest.raises(IndexError):
        m.set_active_blocks(torch.tensor([0, 9]))
    m.train()
    with pytest.raises(RuntimeError, match="ROCm GPU"):  # no CPU path, training included
        m(torch.randn(2, 3, 128))


def test_load_foveal_pattention_mlps_from_safetensors(fsi, tmp_path):
    """A local Llama-style checkpoint (sharded safetensors + index) becomes one
    FovealPattentionMLP per layer with the exact dense weights (K_gate = W_gate,
    K_up = W_up, V = W_down^T over down_proj's storage) and the reference's
    from_dense_mlp router initialisation (zero out_proj)."""
    import json

    import torch
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(0)
    t = {}
    for i in range(3):
        t[f"model.layers.{i}.mlp.gate_proj.weight"] = torch.randn(256, 64, generator=g).bfloat16()
        t[f"model.layers.{i}.mlp.up_proj.weight"] = torch.randn(256, 64, generator=g).bfloat16()
        t[f"model.layers.{i}.mlp.down_proj.weight"] = torch.randn(64, 256, generator=g).bfloat16()
    names = sorted(t)
    shard = {n: ("model-00001-of-00002.safetensors" if "layers.0" in n or "layers.1.mlp.up" in n
                 else "model-00002-of-00002.safetensors") for n in names}
    for f in set(shard.values()):
        save_file({n: t[n] for n in names if shard[n] == f}, str(tmp_path / f))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": shard}))
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 64, "intermediate_size": 256,
                                                      "num_hidden_layers": 3}))
    ms = fsi.load_foveal_pattention_mlps(tmp_path, layers=[0, 2], block_size=64, base_blocks=1, remote_blocks=2,
                                         device="cpu")
    assert sorted(ms) == [0, 2]
    for i, m in ms.items():
        assert torch.equal(m.k_gate, t[f"model.layers.{i}.mlp.gate_proj.weight"])
        assert torch.equal(m.k_up, t[f"model.layers.{i}.mlp.up_proj.weight"])
        assert torch.equal(m.v, t[f"model.layers.{i}.mlp.down_proj.weight"].t()) and m.v.t().is_contiguous()
        assert torch.equal(m.offsets, torch.arange(64)) and not m.out_proj_16d.weight.any()
        assert m.q_proj_16d.weight.dtype == torch.bfloat16 and m.q_proj_16d.weight.std() > 0
        assert m.num_blocks == 4 and m.total_active_blocks == 3
    with pytest.raises(IndexError):
        fsi.load_foveal_pattention_mlps(tmp_path, layers=[3], device="cpu")
    with pytest.raises(KeyError):
        fsi.load_foveal_pattention_mlps(tmp_path, layers=[0], device="cpu", layer_prefix="transformer.h.")
