"""The C-ABI library loads and exports every entry point the header declares
(CPU-only: no kernel is launched).  Argument errors are reported through the
status code and forge_last_error() before any device work."""
import ctypes
import re
from pathlib import Path

import pytest

from forge_hip import _lib as L

HEADER = Path(__file__).resolve().parents[1] / "include" / "forge_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(forge_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "forge_swiglu_fwd" in names and "forge_lora_qkv_rope" in names
    assert len(names) >= 13


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(L.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared in forge_hip.h but not exported: {missing}"
    assert sorted(L.EXPORTED) == sorted(_declared())


def test_identity():
    assert L.forge_version().startswith(b"forge-hip")


def test_arch_check_reports_no_device_without_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: covered by test_arch_check_on_the_gpu")
    assert L.forge_arch_ok() == 0


@pytest.mark.gpu
def test_arch_check_on_the_gpu():
    import torch

    torch.cuda.init()
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert L.forge_arch_ok() == (1 if name.startswith("gfx950") else 0)


def test_status_codes_and_messages():
    # unsupported dtype is rejected before any launch
    rc = L.forge_swiglu_fwd(99, 16, 16, 8, 16, 8, 4, 8, 1.0, 1.0, None)
    assert rc == 2 and b"dtype" in L.forge_last_error()
    rc = L.forge_swiglu_fwd(0, 16, 16, 4, 16, 8, 4, 8, 1.0, 1.0, None)  # ld < cols
    assert rc == 1
    rc = L.forge_rope(2, *([16, 0, 0, 0] * 4), *([16, 0, 0] * 2), 2, 8, None, 1, 4, 3, 8, 127, 0, None)
    assert rc == 1 and b"even" in L.forge_last_error()
    # cos/sin dtype other than q's or fp32; too few table rows without positions
    rc = L.forge_rope(2, *([16, 0, 0, 0] * 4), *([16, 0, 0] * 2), 1, 8, None, 1, 4, 2, 8, 128, 0, None)
    assert rc == 2 and b"cos/sin dtype" in L.forge_last_error()
    rc = L.forge_rope(2, *([16, 0, 0, 0] * 4), *([16, 0, 0] * 2), 2, 7, None, 1, 4, 2, 8, 128, 0, None)
    assert rc == 1 and b"7 rows" in L.forge_last_error()
    rc = L.forge_ce_fwd(2, 16, 4, 2, 8, 16, 1, None, None, None, None, None, -100, *([0.0] * 6), 0, None, None)
    assert rc == 1 and b"ld" in L.forge_last_error()
    rc = L.forge_lora_qkv_rope(16, 64, 100, 256, 0, *([16] * 20)[:14], 16, 16, 8, 16, None, 96, 1, None)
    assert rc == 2
    rc = L.forge_lora_qkv_rope(16, 64, 256, 256, 0, *([16] * 20)[:14], 16, 16, 8, 15, None, 128, 1, None)
    assert rc == 1 and b"15 rows" in L.forge_last_error()
    # an unknown gated activation of the fused LoRA-MLP entry points
    rc = L.forge_lora_mlp_gate_up(16, 64, 64, 0, *([16] * 13), 64, 3, None)
    assert rc == 1 and b"activation 3" in L.forge_last_error()
    rc = L.forge_lora_mlp_down_bwd(16, 64, 64, 0, *([16] * 8), 0, *([16] * 3), 64, -1, None)
    assert rc == 1 and b"activation -1" in L.forge_last_error()


def test_lora_mlp_rank_product_argument_errors():
    """The entry points whose epilogues also form LoRA products check their
    partial-sum buffers, ranks, pitches and alignment before any launch."""
    # forge_lora_mlp_gate_up_v(M, H, I, r, x, ldx, wg, wu, ldw, xa, ld_xa, bg, bu, ldb, e, g, h, ld_out, act,
    #                          a_down, ld_ad, rd, v_part, stream)
    gate_up = [16, 64, 64, 0, 16, 64, 32, 48, 64, None, 0, None, None, 0, 64, 80, 96, 64, 0]
    assert L.forge_lora_mlp_gate_up_v(*gate_up, 112, 64, 16, None, None) == 1
    assert b"v_part is NULL" in L.forge_last_error()
    assert L.forge_lora_mlp_gate_up_v(*gate_up, 112, 64, 4, 128, None) == 1      # rank 4
    assert b"rank 4" in L.forge_last_error()
    assert L.forge_lora_mlp_gate_up_v(*gate_up, 120, 64, 16, 128, None) == 1     # A_down misaligned
    assert b"16-byte aligned" in L.forge_last_error()
    # forge_lora_mlp_down_bwd_v(M, H, I, r, dy, lddy, wd_t, ldwd, t_d, ld_t, ad_t, ld_ad, h, e, g, ld, act,
    #                           bu_t, bg_t, ld_bt, rv, v_part, xa_t_up, xa_t_gate, ld_xat, w_part, stream)
    down = [16, 64, 64, 0, 16, 64, 32, 64, None, 0, None, 0, 48, 64, 80, 64, 0, 96, 112, 64]
    assert L.forge_lora_mlp_down_bwd_v(*down, 16, None, None, None, 0, None, None) == 1
    assert b"v_part is NULL" in L.forge_last_error()
    assert L.forge_lora_mlp_down_bwd_v(*down, 72, 128, None, None, 0, None, None) == 1   # rank 72
    assert b"rank 72" in L.forge_last_error()
    assert L.forge_lora_mlp_down_bwd_v(*down, 16, 128, 152, 176, 16, 200, None) == 1  # xa_t_up misaligned
    assert b"xa^T" in L.forge_last_error()
    assert L.forge_lora_mlp_down_bwd_v(*down, 16, 128, 144, 176, 8, 192, None) == 1   # ld_xat < M
    assert b"ld_xat (8)" in L.forge_last_error()


def test_zero_size_calls_are_noops():
    assert L.forge_swiglu_fwd(0, None, None, 0, None, 0, 0, 0, 1.0, 1.0, None) == 0
    assert L.forge_ce_fwd(2, None, 0, 0, 0, None, 1, None, None, None, None, None, -100, *([0.0] * 6), 0, None, None) == 0


def test_copy_argument_errors():
    # misaligned pointers and overlapping ranges are rejected before any launch
    assert L.forge_copy(16, 24, 64, None) == 1 and b"aligned" in L.forge_last_error()
    assert L.forge_copy(16, 32, 64, None) == 1 and b"overlap" in L.forge_last_error()
    assert L.forge_copy(None, None, 0, None) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes", [1, 15, 16, 4096 + 7, 512 * 16 * 3 + 5, (1 << 24) + 9, (1 << 30) + 16 * 300 + 3])
def test_copy_is_exact(nbytes):
    import torch

    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(nbytes + 16, dtype=torch.uint8, device="cuda")
    L.check(L.forge_copy(dst.data_ptr(), src.data_ptr(), nbytes, L.stream_of(src)), "forge_copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].sum()) == 0  # nothing written past the end
