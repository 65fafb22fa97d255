"""The C-ABI library loads and exports every symbol include/ei_attn.h declares (CPU only:
no compute call needs a GPU here; host-only entry points and argument checks are run)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from tests.parity import bits_equal

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    """Every function the headers under include/ declare."""
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        names |= set(re.findall(r"\b(ei_[a-z0-9_]+)\s*\(", h.read_text()))
    return sorted(names)


def test_header_and_binding_agree():
    from exactinfer_amd import _capi
    assert sorted(_capi.EXPORTS) == _declared()


def test_library_exports_every_declared_symbol():
    from exactinfer_amd import _capi
    L = _capi.lib()
    for name in _declared():
        assert isinstance(getattr(L, name), ctypes._CFuncPtr), name
    header = int(re.search(r"#define EI_ABI_VERSION (\d+)", (ROOT / "include" / "ei_attn.h").read_text()).group(1))
    assert L.ei_abi_version() == header == _capi.ABI_VERSION == 3


def test_rope_table_fill_host_matches_oracle(orc):
    from exactinfer_amd import _capi
    for n_ctx, rd, th in ((64, 128, 1e6), (10, 64, 1e4)):
        out = np.empty((n_ctx, rd // 2, 2), np.float32)
        _capi.call("ei_rope_table_fill", out.ctypes.data, n_ctx, rd, th)
        assert bits_equal(out, orc.rope_table(n_ctx, rd, th))


def test_argument_errors_are_reported_not_thrown():
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="head_dim 64"):
        _capi.call("ei_attn_prefill", None, p, 4096, p, p, p, p, 8, 32, 8, 64, 0.1)
    with pytest.raises(_capi.EiError, match="GQA group 16"):
        _capi.call("ei_attn_prefill", None, p, 4096, p, p, p, p, 8, 128, 8, 128, 0.1)
    with pytest.raises(_capi.EiError, match="multiple of n_head_kv"):
        _capi.call("ei_attn_decode", None, p, p, p, p, p, 30, 8, 128, 0.1, 10, p, 1 << 20)
    with pytest.raises(_capi.EiError, match="workspace"):
        _capi.call("ei_attn_decode", None, p, p, p, p, p, 32, 8, 128, 0.1, 4096, p, 16)
    with pytest.raises(_capi.EiError, match="aligned"):
        _capi.call("ei_kv_append", None, ctypes.c_void_p(18), p, 1024, 1, p, p, 1024, p)
    with pytest.raises(_capi.EiError, match="rope_dim"):
        _capi.call("ei_headnorm_rope", None, p, 1, 4096, 32, 128, p, p, p, 130, 1e-6)
    assert "rope_dim" in _capi.last_error()


def test_shape_limits_are_reported():
    """Shapes past what the size and index arithmetic holds are rejected, not wrapped: more than 1024
    KV heads, prefill chunks past 2^20 tokens or 2^28 query rows, decode grids past 2^31 workgroups;
    the size queries return 0 for them."""
    from exactinfer_amd import _capi
    L = _capi.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="n_head_kv 2048 above 1024"):
        _capi.call("ei_attn_prefill", None, p, 1 << 22, p, p, p, p, 8, 4096, 2048, 128, 0.1)
    assert L.ei_attn_decode_ws_bytes(1, 4096, 2048, 4096) == 0
    assert L.ei_attn_decode_ws_bytes(65536, 32, 8, 4096) == 0
    with pytest.raises(_capi.EiError, match="2\\^20 tokens"):
        _capi.call("ei_attn_prefill", None, p, 4096, p, p, p, p, (1 << 20) + 1, 32, 8, 128, 0.1)
    with pytest.raises(_capi.EiError, match="2\\^28 query rows"):
        _capi.call("ei_attn_prefill_split", None, p, 1 << 20, p, p, p, p, 1 << 20, 512, 64, 128, 0.1, 1 << 20, p,
                   1 << 40)
    assert L.ei_attn_prefill_ws_bytes(1 << 20, 512, 64, 1 << 20) == 0
    with pytest.raises(_capi.EiError, match="more workgroups than one launch takes"):
        _capi.call("ei_attn_decode_batched", None, p, 1 << 20, p, p, p, p, p, 65535, 8192, 1024, 128, 0.1, 1 << 20,
                   p, 1 << 50)


def test_decode_workspace_size_is_monotone():
    from exactinfer_amd import _capi
    L = _capi.lib()
    a = L.ei_attn_decode_ws_bytes(1, 32, 8, 4096)
    b = L.ei_attn_decode_ws_bytes(1, 32, 8, 32768)
    c = L.ei_attn_decode_ws_bytes(64, 16, 8, 8192)
    assert 0 < a <= b and c > 0
    assert L.ei_attn_decode_ws_bytes(1, 30, 8, 10) == 0


def test_prefill_split_workspace_contract():
    from exactinfer_amd import _capi
    L = _capi.lib()
    # chunks of one row over one cache row never split: no workspace
    assert L.ei_attn_prefill_ws_bytes(1, 32, 8, 1) == 0
    # a 512-token chunk with up to 2048 cache rows splits its key range
    a = L.ei_attn_prefill_ws_bytes(512, 32, 8, 2048)
    assert a > 0
    # the size serves every chunk of up to max_B rows, so it never shrinks as max_B grows
    sizes = [L.ei_attn_prefill_ws_bytes(m, 32, 8, 4096) for m in (1, 32, 100, 256, 512, 1024)]
    assert all(x <= y for x, y in zip(sizes, sizes[1:]))
    assert L.ei_attn_prefill_ws_bytes(0, 32, 8, 2048) == 0
    assert L.ei_attn_prefill_ws_bytes(512, 30, 8, 2048) == 0
    assert L.ei_attn_prefill_ws_bytes(512, 32, 8, 100) == 0  # max_kv < max_B
    # one 2048-token chunk: G = 4 fills the CUs unsplit (256 workgroups); G = 2 gives half as many
    # workgroups, so the plan splits its keys (a workspace is needed even at max_B = 2048 alone)
    rows = lambda B, H: B * H
    g4 = L.ei_attn_prefill_ws_bytes(2048, 32, 8, 2048)
    g2 = L.ei_attn_prefill_ws_bytes(2048, 16, 8, 2048)
    assert g2 >= 2 * rows(2048, 16) * 128 * 4  # at least two shares of every (row, head)
    assert g4 > 0  # smaller chunks up to 2048 split
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="workspace"):
        _capi.call("ei_attn_prefill_split", None, p, 4096, p, p, p, p, 512, 32, 8, 128, 0.1, 2048, p, 16)
    with pytest.raises(_capi.EiError, match="max_kv"):
        _capi.call("ei_attn_prefill_split", None, p, 4096, p, p, p, p, 512, 32, 8, 128, 0.1, 100, p, 1 << 30)


def test_prefill_step_argument_errors():
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    args = dict(row_stride=6144, B=512, H=32, HKV=8, D=128, rope_dim=128, max_kv=2048, ws_bytes=1 << 30)

    def call(**kw):
        a = {**args, **kw}
        return _capi.call("ei_prefill_step", None, p, a["row_stride"], p, p, p, p, a["B"], a["H"], a["HKV"], a["D"],
                          p, p, p, a["rope_dim"], 1e-6, 0.1, a["max_kv"], p, a["ws_bytes"])
    with pytest.raises(_capi.EiError, match="rope_dim 130"):
        call(rope_dim=130)
    with pytest.raises(_capi.EiError, match="row_stride"):
        call(row_stride=4096)
    with pytest.raises(_capi.EiError, match="max_kv"):
        call(max_kv=100)
    with pytest.raises(_capi.EiError, match="workspace"):
        call(ws_bytes=16)
    with pytest.raises(_capi.EiError, match="GQA group 16"):
        call(H=128)


def test_paged_argument_errors():
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="block_size 24"):
        _capi.call("ei_attn_decode_paged", None, p, 4096, p, p, p, p, 8, 24, p, 2, 32, 8, 128, 0.1, 128, p, 1 << 20)
    with pytest.raises(_capi.EiError, match="does not cover max_kv"):
        _capi.call("ei_attn_decode_paged", None, p, 4096, p, p, p, p, 4, 16, p, 2, 32, 8, 128, 0.1, 128, p, 1 << 20)
    with pytest.raises(_capi.EiError, match="block_table and kv_len"):
        _capi.call("ei_attn_decode_paged", None, p, 4096, p, p, p, None, 8, 16, p, 2, 32, 8, 128, 0.1, 128, p, 1 << 20)
    with pytest.raises(_capi.EiError, match="exceeds 2"):  # a table spanning more keys than 32-bit indices reach
        _capi.call("ei_attn_decode_paged", None, p, 4096, p, p, p, p, 1 << 26, 64, p, 2, 32, 8, 128, 0.1, 128, p,
                   1 << 20)


def test_fused_decode_rope_dim_multiple_of_4():
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="rope_dim 126"):
        _capi.call("ei_decode_step", None, p, 6144, p, p, p, None, None, p, 1, 32, 8, 128, p, p, p, 126, 1e-6, 0.1,
                   4096, p, 1 << 30)
    with pytest.raises(_capi.EiError, match="rope_dim 62"):
        _capi.call("ei_decode_step_paged", None, p, 6144, p, p, p, p, 8, 16, p, 1, 32, 8, 128, p, p, p, 62, 1e-6,
                   0.1, 128, p, 1 << 30)


def test_projection_rows_per_launch():
    """ei_qkv_project_max_rows: min(4, 24576 / n_embd), the limit HipAttention::project splits by."""
    from exactinfer_amd import _capi
    L = _capi.lib()
    assert [L.ei_qkv_project_max_rows(e) for e in (1024, 2560, 5120, 6144, 8192, 10240, 24577, 0, -5)] == \
        [4, 4, 4, 4, 3, 2, 0, 0, 0]
