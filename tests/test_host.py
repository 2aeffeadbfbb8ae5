"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol include/macai_gdr.h declares
with the argument counts the binding uses, rejects bad arguments with the documented codes before any launch, and the
Python layer's refusals, launch policy and installer (reference tests/test_harness.py:169-173, test_chunking.py:176-199,
patch.py:33-98)."""
import os
import re

import pytest
import torch

from macai.gated_delta import _native as N
from macai.gated_delta import chunk_gated_delta_rule, op
from oracle import gdr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "macai_gdr.h")


def _declared():
    """(name, number of parameters) of every function the header declares."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int64_t|int|const char\s*\*)\s+(macai_gdr_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_library_exports_every_declared_symbol():
    decl = _declared()
    assert {"macai_gdr_prep", "macai_gdr_state_fwd", "macai_gdr_state_bwd", "macai_gdr_state_pair",
            "macai_gdr_chunk_bwd", "macai_gdr_decode", "macai_gdr_group_sum", "macai_gdr_last_error",
            "macai_gdr_abi_version", "macai_gdr_conv_fwd", "macai_gdr_conv_bwd", "macai_gdr_conv_partials",
            "macai_gdr_gates_fwd", "macai_gdr_gates_bwd"} <= set(decl)
    lib = N.lib()
    for name in decl:
        assert hasattr(lib, name), name
    for name, args in N.SIGNATURES.items():
        assert decl[name] == len(args), (name, decl[name], len(args))
    assert lib.macai_gdr_abi_version() == N.ABI_VERSION


def _prep(**over):
    p = 1 << 20
    a = dict(q=p, k=p, v=p, g=p, beta=p, W=p, U=p, Ke=p, GL=p, Qg=p, M=p, A=None, B=1, T=64, H=1, Hk=1, DK=128,
             DV=128, dtype=1, l2=1, scale=1.0, pack=None, NT=0, stream=None)
    a.update(over)
    return N.lib().macai_gdr_prep(*a.values())


def test_abi_rejects_bad_arguments_before_launch():
    L = N.lib()
    assert _prep(DK=96) == N.EUNSUP and b"key head width" in L.macai_gdr_last_error()
    assert _prep(DK=256) == N.EUNSUP and b"256 takes float32" in L.macai_gdr_last_error()   # bf16 at width 256
    assert _prep(DV=48) == N.EUNSUP and b"value head width" in L.macai_gdr_last_error()
    assert _prep(dtype=7) == N.EUNSUP
    assert _prep(T=0) == N.EINVAL
    assert _prep(k=None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert _prep(Ke=None) == N.EINVAL
    assert _prep(M=None) == N.EINVAL
    assert _prep(W=(1 << 20) + 4) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    assert _prep(A=(1 << 20) + 8) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    assert _prep(q=None) == N.EINVAL
    # key heads must divide value heads
    assert _prep(H=4, Hk=3) == N.EINVAL and b"key heads must divide" in L.macai_gdr_last_error()
    assert _prep(H=4, Hk=0) == N.EINVAL
    p = 1 << 20
    sf = lambda *ptrs, flags=0, split=0, DV=128: L.macai_gdr_state_fwd(*ptrs, 1, 64, 1, 128, DV, 1, flags, split,
                                                                       None, 0, None)
    # flags that ask for nothing or carry unknown bits, output + states without the state buffers, a split that does
    # not divide DV / 16, a missing output operand
    assert sf(p, p, p, p, p, p, None, p, None, None, None, flags=8) == N.EINVAL
    assert sf(p, p, p, p, p, p, None, p, None, p, p, flags=2) == N.EINVAL and b"flags" in L.macai_gdr_last_error()
    assert sf(p, p, p, p, p, p, None, p, None, None, p, flags=1) == N.EINVAL and b"Sc" in L.macai_gdr_last_error()
    assert sf(p, p, p, p, p, p, None, p, None, None, None, split=3) == N.EINVAL and b"split" in L.macai_gdr_last_error()
    assert sf(p, p, p, p, p, p, None, p, None, None, None, split=1, DV=96) == N.EINVAL
    assert sf(p, p, p, p, p, None, None, p, None, None, None) == N.EINVAL
    assert L.macai_gdr_state_bwd(p, p, p, p, p, None, None, p, p, p, 1, 64, 1, 128, 128, 1, 0, None, 0,
                                 None) == N.EINVAL
    assert L.macai_gdr_chunk_bwd(*([p] * 15), None, 1, 64, 1, 1, 128, 128, 1, 1, 1.0, None, 0, None) == N.EINVAL
    assert L.macai_gdr_chunk_bwd(*([p] * 16), 1, 64, 6, 4, 128, 128, 1, 1, 1.0, None, 0, None) == N.EINVAL
    pair = lambda *ptrs, split=0: L.macai_gdr_state_pair(*ptrs, 1, 64, 1, 128, 128, 1, split, None, 0, None)
    assert pair(*([p] * 6), None, p, None, p, p, p, p, None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert pair(*([p] * 6), None, p, None, *([p] * 5), split=3) == N.EINVAL
    assert L.macai_gdr_decode(p, p, p, p, p, p, p, p, 1, 1, 1, 256, 128, 1, 1, 1.0, None) == N.EUNSUP
    assert L.macai_gdr_decode(p, p, p, p, p, p, p, p, 1, 4, 3, 128, 128, 1, 1, 1.0, None) == N.EINVAL
    # the segment maps and their scan: null or misaligned buffers, a split giving no valid wave count over DK + DV
    # columns, widths and counts out of range
    sm = lambda *ptrs, split=0, DK=128, DV=128, dtype=1: L.macai_gdr_state_map(*ptrs, 2, 640, 2, DK, DV, dtype, split,
                                                                               None, 0, None)
    assert sm(p, p, p, p, None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert sm(p, p, p + 4, p, p) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    assert sm(p, p, p, p, p, split=3) == N.EINVAL and b"split" in L.macai_gdr_last_error()
    assert sm(p, p, p, p, p, DK=96) == N.EUNSUP and b"float32" in L.macai_gdr_last_error()   # bf16: 32, 64, 128
    assert sm(p, p, p, p, p, DK=256) == N.EUNSUP                       # wide keys take float32 operands
    assert sm(p, p, p, p, p, DK=80, dtype=0) == N.EUNSUP and b"multiple of 32" in L.macai_gdr_last_error()
    assert sm(p, p, p, p, p, DK=288, dtype=0) == N.EUNSUP
    sc = lambda maps, s0, starts, rows=1, nseg=4, DK=128, DV=128: L.macai_gdr_state_scan(maps, s0, starts, rows, nseg,
                                                                                          2, DK, DV, None)
    assert sc(p, None, None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert sc(p, p + 8, p) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    assert sc(p, None, p, nseg=0) == N.EINVAL
    assert sc(p, None, p, rows=70000) == N.EINVAL
    assert sc(p, None, p, DK=80) == N.EUNSUP and sc(p, None, p, DK=288) == N.EUNSUP
    assert sc(p, None, p, DV=24) == N.EUNSUP
    gs = lambda x, y, H=4, Hk=2, D=128, dtype=1: L.macai_gdr_group_sum(x, y, 1, 64, H, Hk, D, dtype, None)
    assert gs(p, None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert gs(p, p, Hk=3) == N.EINVAL
    assert gs(p, p, D=12) == N.EUNSUP
    assert gs(p + 4, p) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    # mixed types (bf16 tensors, float32 arithmetic): prep, the state pass and the per-chunk backward take the code --
    # with it a key width of 256 is valid, so their next check (a null pointer) is what refuses; the per-chunk backward
    # also refuses grouped heads with it; the other entry points refuse the code itself
    B3 = N.BF16_F32
    assert _prep(dtype=B3, DK=256, k=None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert L.macai_gdr_state_fwd(p, p, p, p, p, None, None, p, None, None, None, 1, 64, 1, 256, 128, B3, 0, 0, None, 0,
                                 None) == N.EINVAL
    assert L.macai_gdr_chunk_bwd(*([p] * 15), None, 1, 64, 1, 1, 256, 128, B3, 1, 1.0, None, 0, None) == N.EINVAL
    assert L.macai_gdr_chunk_bwd(*([p] * 16), 1, 64, 4, 2, 128, 128, B3, 1, 1.0, None, 0, None) == N.EUNSUP
    assert b"Hk == H" in L.macai_gdr_last_error()
    assert L.macai_gdr_state_bwd(p, p, p, p, p, p, None, p, p, p, 1, 64, 1, 128, 128, B3, 0, None, 0,
                                 None) == N.EUNSUP
    assert L.macai_gdr_state_pair(*([p] * 6), None, p, None, *([p] * 5), 1, 64, 1, 128, 128, B3, 0, None, 0,
                                  None) == N.EUNSUP
    assert gs(p, p, dtype=B3) == N.EUNSUP


def test_forward_workspace_and_checks():
    """macai_gdr_forward's workspace is the layout the Python host carves for the forward (prep's W, U, Ke, GL, Qg, M,
    each on a 256-byte boundary); a short, misaligned or missing workspace is refused before any launch, and so are
    the shapes macai_gdr_prep refuses."""
    from macai.gated_delta import op
    L = N.lib()
    for (B, T, H, DK, DV, dt, nt) in [(4, 1024, 16, 128, 128, 1, 0), (2, 100, 3, 64, 32, 0, 0), (1, 300, 2, 128, 96, 1, 7)]:
        es = 4 if dt == 0 else 2
        Bc, NT = (1, nt) if nt else (B, -(-T // 64))
        want = op._layout((Bc, H, NT, DK, DV, es, True, False, False, False))[1]
        assert L.macai_gdr_forward_workspace(B, T, H, DK, DV, dt, nt) == want
    p = 1 << 20
    need = L.macai_gdr_forward_workspace(1, 64, 1, 128, 128, 1, 0)
    fw = lambda ws, nbytes, DK=128: L.macai_gdr_forward(p, p, p, p, p, None, p, None, ws, nbytes, 1, 64, 1, 1, DK,
                                                        128, 1, 1, 1.0, 0, None, 0, None)
    assert fw(p, need - 1) == N.EINVAL and b"needs" in L.macai_gdr_last_error()
    assert fw(p + 16, need) == N.EINVAL and b"256-byte" in L.macai_gdr_last_error()
    assert fw(None, need) == N.EINVAL and b"workspace" in L.macai_gdr_last_error()
    assert fw(p, 1 << 30, DK=96) == N.EUNSUP and b"key head width" in L.macai_gdr_last_error()


def test_producer_abi_rejects_bad_arguments():
    """The convolution path's and the gates' entry points check shapes, dtype codes and pointers before any launch."""
    L = N.lib()
    p = 1 << 20
    conv = lambda *ptrs, C=6144, KD=2048, DK=128, REP=1, DV=128, dt=1, vdt=0, B=1, T=8: L.macai_gdr_conv_fwd(
        *ptrs, B, T, C, KD, DK, REP, DV, dt, vdt, None)
    assert conv(p, p, p, p, p, dt=5) == N.EUNSUP
    assert conv(p, p, p, p, None) == N.EINVAL and b"null" in L.macai_gdr_last_error()
    assert conv(p, p, p, p, p, C=6140) == N.EINVAL                 # not a multiple of 8
    assert conv(p, p, p, p, p, DV=96) == N.EINVAL                  # value_dim not a multiple of the head width
    assert conv(p, p, p, p, p, REP=3) == N.EINVAL and b"REP" in L.macai_gdr_last_error()
    assert conv(p + 8, p, p, p, p) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()
    assert conv(p, p, p, p, p, T=0) == N.EINVAL
    assert L.macai_gdr_conv_bwd(p, p, p, p, p, p, p, None, 1, 8, 6144, 2048, 128, 1, 128, 1, 0, None) == N.EINVAL
    assert L.macai_gdr_conv_partials(2, 33, 6144) == 2 * 1 * 6144 * 4      # tiles of 64 time steps
    assert L.macai_gdr_conv_partials(2, 130, 6144) == 2 * 3 * 6144 * 4
    assert L.macai_gdr_gates_fwd(p, p, p, p, p, p, 30, 16, 1, None) == N.EINVAL     # n not a multiple of H
    assert L.macai_gdr_gates_fwd(p, p, p, p, p, p, 32, 16, 9, None) == N.EUNSUP
    assert L.macai_gdr_gates_bwd(p, p, p, p, p, p, p, p, p, None, 32, 16, 1, None) == N.EINVAL


def test_call_maps_codes_to_exceptions():
    with pytest.raises(NotImplementedError, match="key head width"):
        N.call("macai_gdr_prep", *([1 << 20] * 11), None, 1, 64, 1, 1, 96, 128, 1, 1, 1.0, None, 0, None)
    with pytest.raises(ValueError, match="null"):
        N.call("macai_gdr_prep", *([None] * 12), 1, 64, 1, 1, 128, 128, 1, 1, 1.0, None, 0, None)


def test_packed_row_table():
    """cu_seqlens -> the packed-row table of include/macai_gdr.h: each sequence chunked on its own (a 64-token chunk
    never crosses a boundary), empty sequences own no chunk, the last entry is the chunk count."""
    table, NT, N_ = op._pack(torch.tensor([0, 130, 130, 194, 200]), 200, "cpu")
    assert (NT, N_) == (5, 4)
    t0, end, c0 = table[:NT].tolist(), table[NT:2 * NT].tolist(), table[2 * NT:].tolist()
    assert t0 == [0, 64, 128, 130, 194] and end == [130, 130, 130, 194, 200] and c0 == [0, 3, 3, 4, 5]
    assert table.dtype == torch.int32


def test_packed_rows_validated():
    """cu_seqlens must rise from 0 to T; checked before any device work (the reference refused it altogether,
    op.py:270-273)."""
    x = torch.zeros(1, 4, 1, 128)
    for bad in ([0, 2, 3], [1, 4], [0, 3, 2, 4], [0]):
        with pytest.raises(ValueError, match="cu_seqlens"):
            chunk_gated_delta_rule(x, x, x, x[..., 0], x[..., 0], cu_seqlens=torch.tensor(bad))


def test_packed_row_arguments_checked_by_the_abi():
    L = N.lib()
    p = 1 << 20
    # the chunk count must lie in [1, T]; the table must be 4-byte aligned
    assert _prep(pack=p, NT=0) == N.EINVAL and b"packed rows" in L.macai_gdr_last_error()
    assert _prep(pack=p, NT=65) == N.EINVAL
    assert _prep(pack=p + 2, NT=1) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()


def test_cpu_tensors_refused_loudly():
    """No CPU fallback: the product path raises on tensors that are not on a HIP device."""
    x = torch.zeros(1, 4, 1, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        chunk_gated_delta_rule(x, x, x, x[..., 0], x[..., 0])


def test_calls_without_tokens_still_need_the_device():
    """A call without tokens (B = 0 or T = 0) returns at once on the GPU (tests/test_gpu_dropin.py), but off a HIP
    device it is refused like any other."""
    for x in (torch.zeros(2, 0, 2, 64), torch.zeros(0, 3, 2, 64)):
        with pytest.raises(RuntimeError, match="HIP device"):
            chunk_gated_delta_rule(x, x, x, x[..., 0], x[..., 0], output_final_state=True)


def test_split_rule():
    """VALUE_SPLIT 'auto': the largest valid split (1, 2, 4 or 8 waves of 16 columns per workgroup; 8 only when
    nothing else is valid) whose workgroups fit the pass's share of the 256 CUs at once, else the smallest; an int
    setting rounds down to a valid split (reference op.split_for semantics, test_chunking.py:176-199)."""
    assert op.valid_splits(128) == [1, 2, 4, 8] and op.valid_splits(96) == [3, 6] and op.valid_splits(32) == [1, 2]
    assert op.split_for(64, 1024, 128) == 4
    assert op.split_for(16, 32768, 128) == 8
    assert op.split_for(512, 1024, 128) == 2        # never 8 waves of columns when "auto" has another choice
    assert op.split_for(2048, 1, 128) == 2
    assert op.split_for(256, 1024, 128, 2) == 2
    assert op.split_for(4096, 1, 64) == 1           # 4 waves
    assert op.split_for(1, 64, 32) == 2
    assert op.split_for(2, 130, 96) == 6
    assert op.split_for(64, 1024, 128, 2) == 2      # a pass on half the chip (the backward's overlapped passes)
    assert op.split_for(16, 32768, 128, 2) == 8
    old = op.VALUE_SPLIT
    try:
        op.VALUE_SPLIT = 3
        assert op.split_for(64, 1024, 128) == 2
        op.VALUE_SPLIT = 16
        assert op.split_for(64, 1024, 128) == 8
        op.VALUE_SPLIT = 1
        assert op.split_for(64, 1024, 96) == 3
    finally:
        op.VALUE_SPLIT = old


def test_segment_rule():
    """SEQUENCE_SPLIT 'auto': only a single unpacked row whose forward saves nothing, and only when its plain pass
    leaves CUs idle (H x DV / 16 <= 128 workgroups); then the largest power of two with P x H <= 128 and >= 32 chunks
    a segment.  An int forces P (capped at the chunk count).  The map pass may take 8 waves of columns a workgroup
    (key heads up to 128): at H = 16, P = 8 its 7 x 16 head-rows of 256 columns take two slices each, one round."""
    assert op.segments_for(1, 32768, 16, 128) == 8
    assert op.segments_for(1, 32768, 32, 128) == 1       # 256 workgroups already: the maps would only add a chain
    assert op.segments_for(1, 32768, 8, 128) == 16
    assert op.segments_for(1, 4096, 16, 128) == 2        # 64 chunks: two segments of 32
    assert op.segments_for(1, 2048, 16, 128) == 1
    assert op.segments_for(2, 32768, 16, 128) == 1
    assert op.segments_for(1, 32768, 16, 128, save=True) == 1
    assert op.segments_for(1, 32768, 16, 128, pack=object()) == 1
    assert op.split_for(7 * 16, 32768, 256, waves=8) == 2
    assert op.split_for(3 * 16, 32768, 256, waves=8) == 4
    assert op.split_for(7 * 16, 32768, 256) == 4        # 4 waves at most: two rounds
    old = op.SEQUENCE_SPLIT
    try:
        op.SEQUENCE_SPLIT = 3
        assert op.segments_for(1, 32768, 32, 128) == 3
        assert op.segments_for(1, 100, 32, 128) == 2
    finally:
        op.SEQUENCE_SPLIT = old


def test_patch_swaps_the_name_and_restores_it():
    mod = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    import macai.patch as patch
    from macai.gated_delta import recurrent_gated_delta_rule
    orig, orig_dec = mod.torch_chunk_gated_delta_rule, mod.torch_recurrent_gated_delta_rule
    with patch.installed(layer=False, training=False, lora=False, decode=True):
        assert mod.torch_chunk_gated_delta_rule is chunk_gated_delta_rule
        assert mod.torch_recurrent_gated_delta_rule is recurrent_gated_delta_rule
    assert mod.torch_chunk_gated_delta_rule is orig and mod.torch_recurrent_gated_delta_rule is orig_dec
    done = patch.install(layer=False, training=False, lora=False)
    try:
        # the reference's return value: the paths of the modules patched (patch.py:33-56)
        assert "transformers.models.qwen3_5.modeling_qwen3_5" in done and all(isinstance(p, str) for p in done)
        assert ("transformers.models.qwen3_5.modeling_qwen3_5", patch.NAME) in patch.swapped()
        assert mod.torch_recurrent_gated_delta_rule is orig_dec
        assert patch.install(layer=False, training=False, lora=False) == []           # idempotent
        assert patch.install(False, False, False, decode=True) == done                # adds the decode name
        assert mod.torch_recurrent_gated_delta_rule is recurrent_gated_delta_rule
    finally:
        patch.uninstall()
    assert mod.torch_chunk_gated_delta_rule is orig and mod.torch_recurrent_gated_delta_rule is orig_dec
    assert patch.swapped() == []
    with pytest.raises(TypeError):
        patch.install(False, False, False, True)       # decode is keyword-only: the fourth position is not taken


def test_patch_takes_the_reference_keywords():
    """The reference's call forms (patch.py:33, 92) work: the rule is installed, the layer / training / LoRA parts
    (absent here) are reported absent by a RuntimeWarning once each and by the *_patches() helpers."""
    mod = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    import warnings

    import macai.patch as patch
    orig = mod.torch_chunk_gated_delta_rule
    patch._warned.clear()
    with pytest.warns(RuntimeWarning, match="layer, training, lora"):
        with patch.installed():
            assert mod.torch_chunk_gated_delta_rule is chunk_gated_delta_rule
            assert patch.layer_patches() == patch.training_patches() == patch.lora_patches() == []
    assert mod.torch_chunk_gated_delta_rule is orig
    with warnings.catch_warnings():
        warnings.simplefilter("error")          # warned once per part: a second install is silent
        patch.install(layer=True, training=True, lora=True)
        patch.uninstall()
    assert mod.torch_chunk_gated_delta_rule is orig


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "mac-ai-engineering_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), f


def test_noalloc_forward_refuses_oversized_shapes_before_any_launch():
    """The fixed scratch's limit is checked on the host, before the device is touched."""
    L = N.lib()
    p = 1 << 20
    assert L.macai_gdr_forward_workspace(8, 4096, 32, 128, 128, 1, 0) > N.NOALLOC_SCRATCH_BYTES
    rc = L.macai_gdr_forward_noalloc(*([p] * 8), 8, 4096, 32, 32, 128, 128, 1, 1, 1.0, 0, None, 0, None)
    assert rc == N.EINVAL and b"fixed" in L.macai_gdr_last_error()
    assert L.macai_gdr_forward_workspace(4, 1024, 16, 128, 128, 1, 0) <= N.NOALLOC_SCRATCH_BYTES


def test_plan_reports_the_launch_choices():
    """op.plan (the reference's op.py:105-113, here this build's choices), consistent with what the GPU tests see run:
    config 1's forward at split 4 on the chain-and-output kernel, its recompute backward's pair pass at split 2 and
    the persistent per-chunk backward; the stored mode's reverse pass; config 3's 8 segments; the float32 path."""
    p = op.plan(4, 1024, 16, 128, 128, save=True)
    assert p["fwd_chunk"] == p["bwd_chunk"] == 64 and p["operands"] == "bf16" and p["prep"] == "prep8"
    assert (p["fwd_split"], p["fwd_state_pass"], p["segments"]) == (4, "state_out", 1)
    assert (p["recompute"], p["bwd_state_passes"], p["bwd_split"], p["chunk_bwd"]) == (True, "pair", 2, "chunk_bwd8xn")
    assert p["bwd_prep"] == "rerun"
    old = op.RECOMPUTE_STATES, op.KEEP_PREP
    try:
        op.RECOMPUTE_STATES = False
        p = op.plan(4, 1024, 16, 128, 128, save=True)
        assert (p["recompute"], p["bwd_state_passes"], p["bwd_split"], p["bwd_prep"]) == (False, "reverse", 4, "kept")
        op.RECOMPUTE_STATES, op.KEEP_PREP = True, True
        p = op.plan(4, 1024, 16, 128, 128, save=True)
        assert (p["recompute"], p["bwd_state_passes"], p["bwd_split"], p["bwd_prep"]) == (True, "pair", 2, "kept")
    finally:
        op.RECOMPUTE_STATES, op.KEEP_PREP = old
    p = op.plan(1, 32768, 16, 128, 128, save=False)
    assert p["segments"] == 8 and "bwd_state_passes" not in p and p["map_split"] >= 1
    assert op.plan(1, 32768, 16, 128, 128, save=True)["segments"] == 1     # a training forward never splits
    p = op.plan(2, 100, 4, 64, 64, save=True, dtype=torch.float32)
    assert (p["operands"], p["prep"], p["fwd_state_pass"], p["chunk_bwd"]) == ("f32", "prep", "state_fwd", "chunk_bwd")
    # float32 operands run the recompute and reverse passes as two launches unless OVERLAP is True
    p = op.plan(4, 1024, 16, 128, 128, save=True, dtype=torch.float32)
    assert (p["bwd_state_passes"], p["bwd_split"]) == ("recompute+reverse", 4)
    old = op.OVERLAP
    try:
        op.OVERLAP = True
        assert op.plan(4, 1024, 16, 128, 128, save=True, dtype=torch.float32)["bwd_state_passes"] == "pair"
        op.OVERLAP = False
        assert op.plan(4, 1024, 16, 128, 128, save=True)["bwd_state_passes"] == "recompute+reverse"
    finally:
        op.OVERLAP = old
    assert op.pairs_states(torch.float16) and op.pairs_states(torch.bfloat16) and not op.pairs_states(torch.float32)
    assert op.plan(1, 100, 2, 256, 128, save=True)["operands"] == "f32"      # wide keys run the float32 kernels
    assert op.plan(4, 100, 2, 128, 128, save=True)["chunk_bwd"] == "chunk_bwd8"   # fewer chunk-heads than CUs
    assert op.plan(4, 1024, 16, 128, 128, save=True, l2norm=False)["operands"] == "f32"   # keys not normalised
    # bf16 tensors on the float32 kernels go as they are (op.MIXED_IO) where the key heads are the value heads
    assert op.plan(4, 1024, 16, 128, 128, save=True, l2norm=False)["mixed_io"]
    assert not op.plan(4, 1024, 16, 128, 128, save=True, l2norm=False, Hk=4)["mixed_io"]
    assert not op.plan(4, 1024, 16, 128, 128, save=True)["mixed_io"]                     # bf16 operands
    assert not op.plan(4, 1024, 16, 128, 128, save=True, dtype=torch.float32)["mixed_io"]


def test_unnormalized_keys_take_the_float32_kernels(monkeypatch):
    """bf16 calls whose keys the kernels do not normalise (use_qk_l2norm_in_kernel=False) compute in float32 unless
    op.BF16_UNNORMALIZED: the bf16 operands' rounding is amplified as beta |k|^2 grows.  The oracle's rounding model
    (the bf16 path's operand classes) on N(0, 1) keys over 200 tokens at DK = 32 moves o by 1.2e-1 on one of six draws
    (seed 501; the others 4e-3 to 9e-3); the same inputs normalised in the kernels stay under 1e-2.  FUSED_NORM = False
    normalises in its eager prologue, not in the kernels, so it takes the float32 kernels too
    (test_fused_norm_switch)."""
    bf, f32 = torch.bfloat16, torch.float32
    assert op.compute_dtype(bf, 128, 128, True, normalized=False) == f32
    assert op.compute_dtype(bf, 128, 128, True, normalized=True) == bf
    monkeypatch.setattr(op, "BF16_UNNORMALIZED", True)
    assert op.compute_dtype(bf, 128, 128, True, normalized=False) == bf
    model = gdr.BF16_PATH
    names = ("query", "key", "value", "g", "beta", "initial_state")
    inp = gdr.make_inputs(2, 200, 1, 2, 32, 32, bf, s0=True, seed=501)
    worst = {}
    for l2 in (False, True):
        o, sT, gr = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"], use_qk_l2norm_in_kernel=l2)
        o2, sT2, gr2 = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"], use_qk_l2norm_in_kernel=l2, rnd=model)
        worst[l2] = max([gdr.rel(o2, o), gdr.rel(sT2, sT)] + [gdr.rel(gr2[n], gr[n]) for n in gr])
    assert worst[False] > 5e-2 and worst[True] < 1e-2, worst


def test_final_state_gradient_takes_the_float32_backward(monkeypatch):
    """The backward of a bf16 call that receives a gradient of the final state runs on the float32 kernels unless
    op.BF16_STATE_GRAD -- q, k, v handed over as bf16 with float32 arithmetic (op.MIXED_IO, key heads = value heads)
    or upcast, dO upcast, dq, dk, dv in bf16 --; without one -- output_final_state=False, or sT left out of the loss,
    whose gradient then arrives as None -- it keeps the bf16 operands.  Both autograd functions, with the launches
    replaced by recorders.  Why: the oracle's rounding model of the bf16 path (which the kernels
    follow to three digits on this draw) over 150 tokens with an N(0, 1) final-state gradient (seed 209) moves dg by
    2.4e-2; the same draw without it stays under 5e-3."""
    import contextlib
    bf, f32 = torch.bfloat16, torch.float32
    seen = []

    def fake_forward(q, k, v, g, beta, s0, l2norm, q_scale, want_sT, pack=None, keep=False, save=True, mixed=False):
        B, T, H, DV = v.shape
        return v.new_zeros(v.shape), (torch.zeros(B, H, q.shape[-1], DV) if want_sT else None), None

    def fake_backward(q, k, v, g, beta, s0, do, dsT, l2norm, q_scale, pack=None, r=None, mixed=False):
        seen.append((q.dtype, k.dtype, v.dtype, do.dtype, dsT is not None, mixed))
        z = torch.zeros_like
        return z(q), z(k), z(v), z(g), z(beta), None if s0 is None else z(s0)

    monkeypatch.setattr(op, "_forward", fake_forward)
    monkeypatch.setattr(op, "_backward", fake_backward)
    monkeypatch.setattr(op, "_on", lambda dev: contextlib.nullcontext())
    monkeypatch.setattr(op, "_check", lambda *a, **kw: None)
    gen = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(1, 96, 2, 64, generator=gen).to(bf).requires_grad_(True) for _ in range(3))
    g, b = -torch.rand(1, 96, 2, generator=gen), torch.rand(1, 96, 2, generator=gen)
    s0 = torch.zeros(1, 2, 64, 64, requires_grad=True)

    def run(fn, with_state_grad):
        seen.clear()
        if fn == "dropin":
            o, sT = op._DropIn.apply(q, k, v, g, b, None, True, 0.125, True, True, None, False)
        else:
            o, sT = op.GatedDeltaRule.apply(q, k, v, g, b, s0, True)
        outs = [o, sT] if with_state_grad else [o]
        torch.autograd.backward(outs, [torch.ones_like(x) for x in outs])
        assert q.grad.dtype == bf and v.grad.dtype == bf
        q.grad = k.grad = v.grad = None
        return seen[0]

    for fn in ("dropin", "rule"):
        assert run(fn, False) == (bf, bf, bf, bf, False, False)        # sT out of the loss: its gradient is None
        assert run(fn, True) == (bf, bf, bf, f32, True, True)          # bf16 tensors, float32 arithmetic
        monkeypatch.setattr(op, "MIXED_IO", False)
        assert run(fn, True) == (f32, f32, f32, f32, True, False)      # upcast
        monkeypatch.setattr(op, "MIXED_IO", True)
        monkeypatch.setattr(op, "BF16_STATE_GRAD", True)
        assert run(fn, True) == (bf, bf, bf, bf, True, False)
        monkeypatch.setattr(op, "BF16_STATE_GRAD", False)
    assert op.plan(4, 1024, 16, 128, 128, True)["state_grad_operands"] == "f32"
    assert op.plan(4, 1024, 16, 128, 128, True, dtype=f32)["state_grad_operands"] == "f32"
    model = gdr.BF16_PATH
    names = ("query", "key", "value", "g", "beta", "initial_state")
    inp = gdr.make_inputs(1, 150, 2, 2, 128, 128, bf, s0=True, seed=209)
    dsT = torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(216)).double()
    for state_grad, lo, hi in ((dsT, 1e-2, 1.0), (None, 0.0, 5e-3)):
        exact = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"], dsT=state_grad)[2]["dg"]
        path = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"], dsT=state_grad, rnd=model)[2]["dg"]
        assert lo <= gdr.rel(path, exact) < hi, state_grad is None


def test_misaligned_inputs_are_copied_not_refused():
    """A contiguous tensor whose start is not 16-byte aligned (a view at an odd offset) reaches the kernels as an
    aligned copy with the same values (the reference's _even, op.py:58-60); an aligned one passes as it is."""
    base = torch.arange(40, dtype=torch.float32)
    x = base[1:33]
    assert x.is_contiguous() and x.data_ptr() % 16 == 4
    y = op._as(x, torch.float32)
    assert y.data_ptr() % 16 == 0 and torch.equal(y, x)
    z = base[4:36]
    assert op._as(z, torch.float32) is z
    h = torch.arange(40, dtype=torch.bfloat16)[3:35]
    assert op._as(h, torch.bfloat16).data_ptr() % 16 == 0 and torch.equal(op._as(h, torch.bfloat16), h)


def test_short_rows_take_the_float32_kernels(monkeypatch):
    """bf16 calls with gradients on rows shorter than op.BF16_MIN_TOKENS (80) compute in float32: dg, dq of a row of a
    few tokens are sums of few, cancelling terms, and dg of a row of about one chunk is small against its terms, so
    the bf16 operands' rounding is not averaged out (a forward without gradients keeps the bf16 kernels: its outputs
    are not affected).  The oracle's rounding model of the bf16 path on a two-token row (B=1, H=1, DK=DV=32, no
    starting state, seed 50217) moves dg by 5.7e-2, on a 64-token row (B=1, H=2, DK=64, DV=128, seed 134086) by
    1.7e-2; the same draws at 80 tokens stay under 1e-2."""
    bf, f32 = torch.bfloat16, torch.float32
    assert op.BF16_MIN_TOKENS == 80
    assert op.compute_dtype(bf, 128, 128, True, tokens=79) == f32
    assert op.compute_dtype(bf, 128, 128, True, tokens=80) == bf and op.compute_dtype(bf, 128, 128, True) == bf
    assert op.plan(1, 64, 2, 128, 128, True)["operands"] == "f32"
    assert op.plan(1, 80, 2, 128, 128, True)["operands"] == "bf16"
    assert op.plan(1, 3, 2, 128, 128, False)["operands"] == "bf16"   # a forward without gradients keeps bf16
    monkeypatch.setattr(op, "BF16_MIN_TOKENS", 0)
    assert op.compute_dtype(bf, 128, 128, True, tokens=1) == bf
    model = gdr.BF16_PATH
    names = ("query", "key", "value", "g", "beta", "initial_state")
    for T, shape, seed, lo, hi in ((2, (1, 32, 32, False), 50217, 5e-2, 1.0), (80, (1, 32, 32, False), 50217, 0.0, 1e-2),
                                   (64, (2, 64, 128, False), 134086, 1e-2, 1.0),
                                   (80, (2, 64, 128, False), 134086, 0.0, 1e-2)):
        H, DK, DV, s0 = shape
        inp = gdr.make_inputs(1, T, H, H, DK, DV, bf, s0=s0, seed=seed)
        exact = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"])[2]["dg"]
        path = gdr.dropin_f64(*(inp[n] for n in names), do=inp["do"], rnd=model)[2]["dg"]
        assert lo <= gdr.rel(path, exact) < hi, (T, seed)


def test_fused_norm_switch(monkeypatch):
    """op.FUSED_NORM (the reference's switch, op.py:19-21): True hands the raw query and key to the kernels with the
    normalisation fused (use_l2norm 1); False normalises them as float32 PyTorch operations (autograd records them)
    and asks the kernels for the scale only (use_l2norm 0), on the float32 kernels with the normalised values kept in
    float32 -- or, with op.BF16_UNNORMALIZED, rounded to bf16."""
    seen = {}

    def fake_apply(q, k, v, g, beta, s0, l2norm, q_scale, want_sT, save, pack, mixed):
        seen.update(q=q, k=k, v=v, l2norm=l2norm, q_scale=q_scale, mixed=mixed)
        return v.new_zeros(v.shape)

    monkeypatch.setattr(op, "_check", lambda *a, **kw: None)
    monkeypatch.setattr(op._DropIn, "apply", staticmethod(fake_apply))
    gen = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 96, 2, 64, generator=gen).to(torch.bfloat16) for _ in range(3))
    g, b = -torch.rand(1, 96, 2, generator=gen), torch.rand(1, 96, 2, generator=gen)
    chunk_gated_delta_rule(q, k, v, g, b, use_qk_l2norm_in_kernel=True)
    assert seen["l2norm"] is True and seen["q"] is q and seen["q_scale"] == 64 ** -0.5
    monkeypatch.setattr(op, "FUSED_NORM", False)
    qr = q.clone().requires_grad_(True)
    chunk_gated_delta_rule(qr, k, v, g, b, use_qk_l2norm_in_kernel=True)
    assert seen["l2norm"] is False and seen["q_scale"] == 64 ** -0.5
    assert seen["q"].dtype == torch.float32 and seen["q"].requires_grad and seen["v"].dtype == torch.float32
    assert torch.equal(seen["q"], op.l2norm(q.float())) and torch.equal(seen["k"], op.l2norm(k.float()))
    assert not seen["mixed"]                  # the normalised q, k are float32 tensors: v is upcast with them
    assert op.plan(1, 96, 2, 64, 64, True)["operands"] == "f32"
    monkeypatch.setattr(op, "BF16_UNNORMALIZED", True)
    chunk_gated_delta_rule(qr, k, v, g, b, use_qk_l2norm_in_kernel=True)
    assert seen["q"].dtype == torch.bfloat16 and seen["q"].requires_grad
    assert torch.equal(seen["q"], op.l2norm(q.float()).to(torch.bfloat16))
    assert torch.equal(seen["k"], op.l2norm(k.float()).to(torch.bfloat16))
    monkeypatch.setattr(op, "BF16_UNNORMALIZED", False)
    chunk_gated_delta_rule(q, k, v, g, b, use_qk_l2norm_in_kernel=False)      # nothing to normalise either way;
    assert seen["l2norm"] is False and seen["mixed"] and seen["q"] is q       # keys of unknown norm: float32 kernels
    monkeypatch.setattr(op, "MIXED_IO", False)                               # (bf16 tensors as they are, or upcast)
    chunk_gated_delta_rule(q, k, v, g, b, use_qk_l2norm_in_kernel=False)
    assert not seen["mixed"] and torch.equal(seen["q"], q.float()) and seen["q"].dtype == torch.float32
    monkeypatch.setattr(op, "MIXED_IO", True)
    monkeypatch.setattr(op, "BF16_UNNORMALIZED", True)
    chunk_gated_delta_rule(q, k, v, g, b, use_qk_l2norm_in_kernel=False)
    assert seen["l2norm"] is False and seen["q"] is q and not seen["mixed"]


def test_gates_and_conv_check_their_arguments():
    """supported() with the reference's signatures (layer/_gates.py:75, layer/_conv.py:178), and the autograd
    functions refusing shapes that would make the kernels read past a tensor or mix up heads, before any launch."""
    from macai.layer import _conv, _gates, conv_qkv, gates
    H = 4
    b, a = torch.randn(2, 3, H), torch.randn(2, 3, H)
    A_log, dt = torch.zeros(H), torch.zeros(H)
    assert not _gates.supported(b, a, A_log, dt)                 # CPU tensors: the kernels run on a HIP device
    assert _gates._unfit(b, a, A_log, dt) is None
    with pytest.raises(RuntimeError, match="HIP device"):
        gates(b, a, A_log, dt)
    bad = [((b, a[:, :2], A_log, dt), "one shape"), ((b, a.double(), A_log, dt), "dtype"),
           ((b, a, A_log[None], dt), r"\[H\]"), ((b, a, A_log, dt[:3]), r"\[H\]"),
           ((torch.randn(2, 3, 5), torch.randn(2, 3, 5), A_log, dt), r"\[H\]"),
           ((b.to(torch.int32), a.to(torch.int32), A_log, dt), "dtype")]
    for args, msg in bad:
        assert _gates._unfit(*args) is not None
        with pytest.raises(ValueError, match=msg):
            gates(*args)
    kd, dk, dv, rep = 32, 16, 16, 2                              # 2 key heads, 4 value heads
    C = 2 * kd + 4 * dv
    x, w = torch.randn(2, 9, C), torch.randn(C, 1, 4)
    assert not _conv.supported(x, w, kd, dk, rep, dv) and _conv._unfit(x, w, kd, dk, rep, dv) is None
    with pytest.raises(RuntimeError, match="HIP device"):
        conv_qkv(x, w, kd, dk, rep, dv)
    bad = [((x[0], w, kd, dk, rep, dv), r"\[B, T, C\]"), ((x, w[:-1], kd, dk, rep, dv), "taps"),
           ((x, w, kd, dk, 3, dv), "key_dim"), ((x, w, 24, 12, rep, dv), "key_dim"),
           ((x.to(torch.int32), w, kd, dk, rep, dv), "float32")]
    for args, msg in bad:
        assert _conv._unfit(*args) is not None
        with pytest.raises(ValueError, match=msg):
            conv_qkv(*args)


def test_mfma_probe_checks_and_counts():
    """The matrix-core probe's FLOP count (2 per multiply-add: 8 chains x iters x 4 waves a workgroup) and its
    argument checks, before any launch."""
    L = N.lib()
    assert L.macai_gdr_probe_mfma_flops(0, 10, 3) == 16384 * 8 * 10 * 3 * 4
    assert L.macai_gdr_probe_mfma_flops(1, 10, 3) == 2048 * 8 * 10 * 3 * 4
    assert L.macai_gdr_probe_mfma_flops(2, 10, 3) == 32768 * 8 * 10 * 3 * 4
    assert L.macai_gdr_probe_mfma_flops(3, 10, 3) == -1
    p = 1 << 20
    assert L.macai_gdr_probe_mfma(3, 10, p, 4, None) == N.EINVAL
    assert L.macai_gdr_probe_mfma(0, 0, p, 4, None) == N.EINVAL
    assert L.macai_gdr_probe_mfma(0, 10, p + 4, 4, None) == N.EINVAL and b"aligned" in L.macai_gdr_last_error()


def test_head_widths():
    """Key widths: every multiple of 32 up to 256 on the float32 kernels, 32 / 64 / 128 on the bf16 ones; value widths
    in the backward: up to 256 on the float32 kernels, 128 on the bf16 ones (the reference takes any multiple of 32,
    op.py:124-125).  bf16 inputs at other widths are computed as float32; widths no kernel takes are refused, on the
    host and by the C ABI before any launch."""
    bf, f32 = torch.bfloat16, torch.float32
    assert op.compute_dtype(bf, 128, 128, True) == bf and op.compute_dtype(bf, 64, 96, True) == bf
    assert op.compute_dtype(bf, 96, 128, True) == f32 and op.compute_dtype(bf, 256, 128, False) == f32
    assert op.compute_dtype(bf, 128, 256, True) == f32          # the bf16 backward stops at value width 128
    assert op.compute_dtype(bf, 128, 256, False) == bf          # a forward alone keeps bf16 operands
    assert op.compute_dtype(torch.float16, 128, 128, True) == f32
    for DK, DV, save in ((96, 256, True), (224, 160, True), (256, 512, False)):
        op._widths(DK, DV, save)
    for DK, DV, save, msg in ((80, 128, False, "key head"), (288, 128, False, "key head"), (128, 48, False, "value"),
                              (128, 288, True, "backward")):
        with pytest.raises(NotImplementedError, match=msg):
            op._widths(DK, DV, save)
    L, p = N.lib(), 1 << 20

    def cb(DK=128, DV=128, dtype=0):
        return L.macai_gdr_chunk_bwd(*([p] * 16), 1, 64, 2, 2, DK, DV, dtype, 1, 1.0, None, 0, None)
    assert cb(DV=160, dtype=1) == N.EUNSUP and b"bf16 backward" in L.macai_gdr_last_error()
    assert cb(DV=288) == N.EUNSUP and b"up to 256" in L.macai_gdr_last_error()
    assert cb(DK=96, dtype=1) == N.EUNSUP and b"float32" in L.macai_gdr_last_error()
    assert cb(DK=80) == N.EUNSUP and b"multiple of 32" in L.macai_gdr_last_error()
