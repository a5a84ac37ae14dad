"""C-ABI and host-side logic (CPU only: no kernel is launched here).

* libsimsd_kernels.so loads and exports every function include/simsd_kernels.h
  declares, with the ABI version the header states;
* the host-only entry points (sizes, plans) agree with the Python mirror of
  the reference's config rules;
* the dispatch envelope and error behaviour of the reference's module
  (kernels/thin_linear_fused_test.py:112-127, 154-195) hold for the drop-in;
* the toggle swaps/restores modules (kernels/thin_linear_fused_test.py:253-298).
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch
import torch.nn as nn

from conftest import REPO

HEADER = os.path.join(REPO, "include", "simsd_kernels.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(simsd_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from kernels import _native
    lib = _native.lib()
    names = header_functions()
    assert len(names) >= 10, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)


def test_abi_version_matches_header():
    from kernels import _native
    m = re.search(r"#define SIMSD_ABI_VERSION (\d+)", open(HEADER).read())
    assert int(m.group(1)) == _native.lib().simsd_abi_version() == _native.ABI_VERSION


def test_header_constants_match_binding():
    from kernels import _native
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (SIMSD_\w+) (\d+)", text))
    assert int(consts["SIMSD_DTYPE_BF16"]) == _native.DTYPE_CODES[torch.bfloat16]
    assert int(consts["SIMSD_DTYPE_F16"]) == _native.DTYPE_CODES[torch.float16]
    assert int(consts["SIMSD_DTYPE_F32"]) == _native.DTYPE_CODES[torch.float32]
    assert int(consts["SIMSD_SCORE_SOFTMAX"]) == _native.SCORE_SOFTMAX
    assert int(consts["SIMSD_SCORE_SIGMOID"]) == _native.SCORE_SIGMOID
    assert int(consts["SIMSD_MOE_MAX_EXPERTS"]) == _native.MOE_MAX_EXPERTS
    assert int(consts["SIMSD_MOE_MAX_SLOTS"]) == _native.MOE_MAX_SLOTS


def test_header_links_from_plain_c(tmp_path):
    """A C program includes the header, links the library and calls the
    host-only entry points (no GPU needed)."""
    from kernels import _native
    src = tmp_path / "t.c"
    src.write_text(
        '#include <stdio.h>\n#include "simsd_kernels.h"\n'
        'int main(void){\n'
        '  int out[4];\n'
        '  if (simsd_abi_version() != SIMSD_ABI_VERSION) return 1;\n'
        '  if (simsd_moe_num_tiles(512, 256) != 288) return 2;\n'
        '  if (simsd_thin_linear_plan(4, 12288, 2048, SIMSD_DTYPE_BF16, 0, 0, 0, out) != 0) return 3;\n'
        '  printf("%d %d %d %d\\n", out[0], out[1], out[2], out[3]);\n'
        '  return 0;\n}\n')
    libdir = os.path.dirname(_native.LIB_PATH)
    exe = tmp_path / "t"
    rc = os.system(f"gcc -std=c99 -Wall -Werror -I{REPO}/include {src} -o {exe} "
                   f"-L{libdir} -lsimsd_kernels -Wl,-rpath,{libdir}")
    assert rc == 0
    assert os.system(f"{exe} > {tmp_path}/out.txt") == 0
    # 16 weight rows per workgroup, the 4-token GEMV column block, 4 waves, no split
    assert open(f"{tmp_path}/out.txt").read().split() == ["16", "4", "4", "1"]


@pytest.mark.parametrize("M,N,K", [(4, 2048, 2048), (4, 1024, 2048), (4, 12288, 2048),
                                   (4, 2048, 6144), (16, 4096, 4096), (32, 24576, 4096),
                                   (32, 4096, 12288), (4, 151936, 2048), (96, 2048, 2048),
                                   (1, 1, 1), (7, 33, 1000), (24, 1024, 4096), (9, 100, 64),
                                   (36, 6144, 4096), (48, 4096, 12288), (40, 100, 64), (49, 4096, 4096)])
def test_c_plan_equals_python_heuristic(M, N, K):
    from kernels import _native
    from kernels.thin_linear_fused import _heuristic_config
    out = (ctypes.c_int * 4)()
    assert _native.lib().simsd_thin_linear_plan(M, N, K, 0, 0, 0, 0, out) == 0
    rows, cols, waves, split = list(out)
    BM, BN, BK, SK = _heuristic_config(M, N, K, 2)
    assert (rows, cols, split) == (BN, BM, SK)
    assert waves == 4


def test_workspace_sizes():
    from kernels import _native
    lib = _native.lib()
    assert lib.simsd_thin_linear_workspace_bytes(4, 2048, 2048, 0, 16, 1, 4) == 0
    n = lib.simsd_thin_linear_workspace_bytes(4, 2048, 6144, 0, 16, 8, 4)
    assert n == 8 * 4 * 2048 * 4          # 8 fp32 partial tiles of 4 x 2048
    assert lib.simsd_thin_linear_workspace_bytes(4, 2048, 6144, 0, 12, 1, 4) == -1   # bad block_n
    assert lib.simsd_moe_num_tiles(512, 256) == 256 + 32
    assert lib.simsd_moe_num_tiles(32, 256) == 32 + 2
    w = lib.simsd_moe_workspace_bytes(64, 8, 2048, 512, 512, 0)
    assert w >= 2 * (512 * 512 + 64 * 512 + 512 * 2048 + 64 * 2048)
    # attention: one workgroup per KV head needs none (16 rows up to 256
    # slots, 32 rows up to 384); the split head form needs 256 bytes of
    # arrival counters, then P partials of 16 (32) rows x 128 fp32 and their
    # (max, sum) per KV head: the most workgroups any valid length up to the
    # bound's n = ceil(slots / 32) key steps takes -- one step a wave (4 waves)
    # up to 28 steps, 1.5 above, at most 8 -- or n + 1 steps' (the fused
    # launch's new keys), whichever is more
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 200) == 0
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 256) == 0
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 512) == 256 + 8 * 5 * 16 * 128 * 4 + 8 * 5 * 16 * 8
    assert lib.simsd_block_attention_workspace_bytes(16, 16, 8, 384) == 0      # 32 rows
    assert lib.simsd_block_attention_workspace_bytes(16, 16, 8, 768) == 256 + 8 * 7 * 32 * 128 * 4 + 8 * 7 * 32 * 8
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 1200) == 256 + 8 * 7 * 16 * 128 * 4 + 8 * 7 * 16 * 8
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 1024) == 256 + 8 * 7 * 16 * 128 * 4 + 8 * 7 * 16 * 8
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 3000) == 256 + 8 * 9 * 16 * 128 * 4 + 8 * 9 * 16 * 8
    # more than 32 rows per KV head, or past 4096 slots: the chunked form
    assert lib.simsd_block_attention_workspace_bytes(36, 32, 8, 1024) > 256
    assert lib.simsd_block_attention_workspace_bytes(4, 16, 8, 5000) > 256
    assert lib.simsd_block_attention_workspace_bytes(4, 12, 8, 100) == -1      # 12 q heads over 8 KV heads


def test_partial_row_tile_plan():
    """block_n = 24 keeps 24 rows per workgroup on the ungated 9..32-token
    kernel (N = 6144: 256 workgroups) and acts as 16 elsewhere."""
    from kernels import _native
    from kernels.thin_linear_fused import _rows_for
    lib = _native.lib()
    out = (ctypes.c_int * 4)()
    assert lib.simsd_thin_linear_plan(16, 6144, 4096, 0, 24, 1, 4, out) == 0
    assert list(out) == [24, 16, 4, 1]
    assert lib.simsd_thin_linear_plan(32, 6144, 4096, 1, 24, 2, 8, out) == 0   # fp16
    assert list(out) == [24, 32, 8, 2]
    assert lib.simsd_thin_linear_plan(4, 6144, 4096, 0, 24, 1, 4, out) == 0    # GEMV
    assert out[0] == 16
    assert lib.simsd_thin_linear_plan(16, 6144, 4096, 2, 24, 1, 4, out) == 0   # fp32
    assert out[0] == 16
    assert _rows_for(24) == 24 and _rows_for(31) == 24 and _rows_for(23) == 16


def test_error_string_round_trip():
    from kernels import _native
    lib = _native.lib()
    st = lib.simsd_thin_linear(None, 0, 0, None, 0, 0, None, 0, None, 0, 0, 4, 4, 4, 9,
                               0, 0, 0, 0, None, 0, None)
    assert st != 0
    assert b"dtype" in lib.simsd_last_error_string()
    with pytest.raises(RuntimeError, match="dtype"):
        _native.check(st, "thin_linear")


# ─────────────────────────────── reference envelope / errors (host only) ───
def test_tuned_table_envelope():
    from kernels.thin_linear_fused import TUNED, _tuned_for, should_fuse, pick_config
    assert (2048, 2048) in TUNED
    assert _tuned_for(4, 2048, 2048) is not None
    assert _tuned_for(16, 2048, 2048) is not None
    assert _tuned_for(96, 2048, 2048) is None
    # range entries inside their token range only, never overlapping
    from kernels.thin_linear_fused import TUNED_RANGES, _ROWS
    for (K, N), ranges in TUNED_RANGES.items():
        assert (K, N) in TUNED
        spans = sorted(r for r, _ in ranges)
        assert all(a[1] < b[0] for a, b in zip(spans, spans[1:]))
        for (lo, hi), cfg in ranges:
            assert 1 <= lo <= hi <= TUNED[(K, N)][0]
            # rows the kernels are built for; at least 16 above 8 tokens
            # (whole 16-row MFMA blocks), GEMV ranges stay within 8 tokens
            assert cfg[1] in _ROWS and (cfg[1] >= 16 if lo > 8 else hi <= 8)
            assert _tuned_for(lo, N, K) == cfg and _tuned_for(hi, N, K) == cfg
            assert _tuned_for(lo - 1, N, K) == TUNED[(K, N)] or any(
                a <= lo - 1 <= b for (a, b), _ in ranges)
        assert _tuned_for(4, N, K) == TUNED[(K, N)]
    assert _tuned_for(8, 4096, 2048) == (16, 16, 256, 1, 4, 2)
    assert _tuned_for(9, 4096, 2048) == TUNED[(2048, 4096)]
    assert _tuned_for(4, 999, 2048) is None
    assert should_fuse(4, 2048, 2048) and should_fuse(16, 2048, 2048)
    assert not should_fuse(32, 2048, 2048) and not should_fuse(96, 2048, 2048)
    # target shapes extend to the verify with committed blocks folded in
    # (up to 48 rows; the envelope is 64), not to prefill
    for K, N in [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096), (4096, 151936)]:
        assert should_fuse(4, N, K) and should_fuse(16, N, K) and should_fuse(32, N, K)
        assert should_fuse(36, N, K) and should_fuse(48, N, K) and should_fuse(64, N, K)
        assert not should_fuse(65, N, K) and not should_fuse(96, N, K)
    assert len(pick_config(4, 2048, 2048)) == 4
    assert pick_config(96, 2048, 2048)[0] == 32


def test_rejects_grad_mode_and_dtype_mismatch_on_host():
    from kernels.thin_linear_fused import thin_linear
    x = torch.randn(4, 64, dtype=torch.bfloat16).requires_grad_(True)
    w = torch.randn(32, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="forward-only"):
        thin_linear(x, w)
    with pytest.raises(TypeError):
        with torch.inference_mode():
            thin_linear(torch.randn(4, 64, dtype=torch.bfloat16), torch.randn(32, 64))
    with pytest.raises(ValueError):
        with torch.inference_mode():
            thin_linear(torch.randn(4, 64, dtype=torch.bfloat16),
                        torch.randn(2, 32, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        with torch.inference_mode():
            thin_linear(torch.randn(4, 64, dtype=torch.bfloat16),
                        torch.randn(32, 63, dtype=torch.bfloat16))


def test_cpu_tensors_fail_loudly():
    """No silent CPU fallback: host tensors are refused."""
    from kernels.thin_linear_fused import thin_linear
    from kernels.moe_dispatch_fused import moe_dispatch, moe_route
    with pytest.raises(RuntimeError, match="device"):
        with torch.inference_mode():
            thin_linear(torch.randn(4, 64, dtype=torch.bfloat16),
                        torch.randn(32, 64, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="device"):
        moe_route(torch.randn(4, 16), 2)
    with pytest.raises(RuntimeError, match="device"):
        moe_dispatch(torch.randn(4, 8), torch.zeros(4, 2, dtype=torch.long),
                     torch.ones(4, 2), torch.randn(3, 4, 8), torch.randn(3, 4, 8),
                     torch.randn(3, 8, 4))


def test_moe_num_tiles_and_block_m():
    from kernels import moe_dispatch_fused as m
    from kernels import _native
    assert m.BLOCK_M == 16
    for M, E in [(1, 256), (32, 256), (512, 256), (256, 8), (7, 13)]:
        assert m._num_tiles(M, E) == _native.lib().simsd_moe_num_tiles(M, E)


# ────────────────────────────────────────────── toggle (host modules) ───
class _Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(512, 512, bias=False)
        self.gate_proj = nn.Linear(512, 1024, bias=False)
        self.other = nn.Linear(512, 8, bias=False)

    def forward(self, x):
        return self.gate_proj(self.q_proj(x)), self.other(x)


def test_toggle_swaps_and_restores_host():
    from kernels import fused_toggle
    from kernels.thin_linear_fused import ThinLinear
    m = _Tiny().eval()
    x = torch.randn(4, 512)
    with torch.inference_mode():
        ref = m(x)
    assert fused_toggle.apply_to_model(m, True) == 2
    assert isinstance(m.q_proj, ThinLinear) and isinstance(m.other, nn.Linear)
    assert fused_toggle.apply_to_model(m, True) == 0
    with torch.inference_mode():
        got = m(x)             # (512, 512) is not a tuned shape -> F.linear
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    assert fused_toggle.apply_to_model(m, False) == 2
    assert isinstance(m.q_proj, nn.Linear) and not fused_toggle.is_applied(m)


def test_toggle_state_dict_aliasing_and_noop_host():
    from kernels import fused_toggle
    m = _Tiny().eval()
    before = {k: v.clone() for k, v in m.state_dict().items()}
    ptr = m.q_proj.weight.data_ptr()
    with fused_toggle.fused_linear(m):
        after = m.state_dict()
        assert set(after) == set(before)
        assert all(torch.equal(after[k], before[k]) for k in before)
        assert m.q_proj.weight.data_ptr() == ptr
    m2 = _Tiny()
    assert fused_toggle.apply_to_model(m2, False) == 0
    assert isinstance(m2.q_proj, nn.Linear)


def test_toggle_lm_head_opt_in():
    from kernels import fused_toggle
    from kernels.thin_linear_fused import ThinLinear

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.o_proj = nn.Linear(8, 8)
            self.lm_head = nn.Linear(8, 16)
    m = M()
    assert fused_toggle.apply_to_model(m, True) == 1
    assert isinstance(m.lm_head, nn.Linear)
    fused_toggle.apply_to_model(m, False)
    assert fused_toggle.apply_to_model(m, True, targets=fused_toggle.ALL_TARGETS) == 2
    assert isinstance(m.lm_head, ThinLinear)
    fused_toggle.apply_to_model(m, False)


class _Expert(nn.Module):
    def __init__(self, H, I):
        super().__init__()
        self.gate_proj = nn.Linear(H, I, bias=False)
        self.up_proj = nn.Linear(H, I, bias=False)
        self.down_proj = nn.Linear(I, H, bias=False)


class LLaDA2MoeSparseMoeBlock(nn.Module):
    """Stand-in with the remote class's name and the moe_infer signature."""

    def __init__(self, E=4, H=16, I=8):
        super().__init__()
        self.experts = nn.ModuleList(_Expert(H, I) for _ in range(E))

    def moe_infer(self, x, topk_ids, topk_weight):
        return "stock"


def test_apply_moe_to_model_host():
    from kernels import fused_toggle
    from kernels.moe_dispatch_fused import stack_expert_weights
    root = nn.Module()
    root.blk = LLaDA2MoeSparseMoeBlock()
    g0 = root.blk.experts[1].gate_proj.weight.detach().clone()
    assert fused_toggle.apply_moe_to_model(root, True) == 1
    assert fused_toggle.is_moe_applied(root)
    wg, wu, wd = fused_toggle.expert_stacks(root.blk)
    assert wg.shape == (4, 8, 16) and wd.shape == (4, 16, 8)
    assert torch.equal(wg[1], g0)
    assert root.blk.experts[1].gate_proj.weight.numel() == 0        # destructive
    assert fused_toggle.apply_moe_to_model(root, True) == 0          # idempotent
    with pytest.raises(NotImplementedError):
        fused_toggle.apply_moe_to_model(root, False)
    # unpatched instances keep the stock method; nothing is patched on the class
    other = LLaDA2MoeSparseMoeBlock()
    assert other.moe_infer(None, None, None) == "stock"
    assert LLaDA2MoeSparseMoeBlock.moe_infer(other, None, None, None) == "stock"
    assert fused_toggle.apply_moe_to_model(nn.Module(), False) == 0   # nothing switched: no error
    ex = nn.ModuleList(_Expert(16, 8) for _ in range(3))
    a, b, c = stack_expert_weights(ex, free_originals=False)
    assert a.is_contiguous() and ex[0].gate_proj.weight.numel() == 128


def test_gated_mlp_toggle_host():
    """apply_gated_mlp_to_model patches SiLU-gated blocks only, is idempotent,
    skips biased gate/up, and restores the class forward."""
    import torch.nn as nn
    from kernels.fused_toggle import apply_gated_mlp_to_model, is_gated_mlp_applied

    class MLP(nn.Module):
        def __init__(self, bias=False, act=None):
            super().__init__()
            self.gate_proj = nn.Linear(16, 8, bias=bias)
            self.up_proj = nn.Linear(16, 8, bias=bias)
            self.down_proj = nn.Linear(8, 16, bias=False)
            self.act_fn = act if act is not None else nn.SiLU()

        def forward(self, x):
            return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))

    model = nn.Sequential(MLP(), MLP(bias=True), MLP(act=nn.GELU()), MLP())
    assert apply_gated_mlp_to_model(model) == 2
    assert is_gated_mlp_applied(model)
    assert "forward" in model[0].__dict__ and "forward" not in model[1].__dict__
    assert "forward" not in model[2].__dict__
    assert apply_gated_mlp_to_model(model) == 0            # idempotent
    assert apply_gated_mlp_to_model(model, enable=False) == 2
    assert not is_gated_mlp_applied(model)
    assert all("forward" not in m.__dict__ for m in model)
    x = torch.randn(3, 16)
    with torch.no_grad():                                   # the stock CPU path is back
        assert model(x).shape == (3, 16)


def test_rmsnorm_toggle_host():
    import torch.nn as nn
    from kernels.fused_toggle import apply_rmsnorm_to_model

    class TinyRMSNorm(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.weight = nn.Parameter(torch.ones(n))
            self.variance_epsilon = 1e-6

        def forward(self, x):
            return x

    model = nn.Sequential(TinyRMSNorm(8), nn.LayerNorm(8), TinyRMSNorm(8))
    assert apply_rmsnorm_to_model(model) == 2
    assert apply_rmsnorm_to_model(model) == 0
    x = torch.randn(2, 8)
    assert torch.equal(model[0](x), x)          # CPU tensors keep the stock forward
    assert apply_rmsnorm_to_model(model, enable=False) == 2
    assert "forward" not in model[0].__dict__


def test_attention_graph_bounds_host():
    """The runner captures one graph per attention bound: steps up to the
    one-launch form's limit, else the whole cache."""
    from kernels.attention_fused import ONE_LAUNCH_SLOTS
    from speculative.step import valid_bound
    assert ONE_LAUNCH_SLOTS == 4096
    assert valid_bound(8000, 500) == 1024
    assert valid_bound(8000, 1024) == 1024
    assert valid_bound(8000, 1025) == 2048
    assert valid_bound(8000, 3500) == 4096
    assert valid_bound(8000, 5000) == 8000
    assert valid_bound(2000, 1800) == 2000
    assert valid_bound(700, 600) == 700


def test_toggle_warmup_and_ledger_host():
    """warmup on CPU modules returns without launching anything; the ledger
    holds the model weakly (a collected model leaves no entry)."""
    import gc
    from kernels import fused_toggle
    m = _Tiny().eval()
    assert fused_toggle.apply_to_model(m, True) == 2
    fused_toggle.warmup(m, block_length=4)           # (512, *) shapes are not tuned -> F.linear on CPU
    assert fused_toggle.is_applied(m)
    n_before = len(fused_toggle._LINEARS._by_model)
    del m
    gc.collect()
    assert len(fused_toggle._LINEARS._by_model) == n_before - 1


def test_accept_blocks_matches_oracle_host():
    """The runner's acceptance equals the oracle's restatement of the
    reference's K-block loop on hand cases and random draws."""
    import random
    from oracle import verify as over
    from speculative.verify import accept_blocks
    cases = [([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 2, 3, 4], [5, 6, 7, 8]]),
             ([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 2, 9, 4], [5, 6, 7, 8]]),
             ([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 2, 3, 4], [0, 6, 7, 8]]),
             ([[1, 2, 3, 4]], [[9, 9, 9, 9]])]
    rng = random.Random(0)
    for _ in range(200):
        K = rng.randint(1, 4)
        d = [[rng.randint(0, 3) for _ in range(4)] for _ in range(K)]
        t = [[rng.randint(0, 3) for _ in range(4)] for _ in range(K)]
        cases.append((d, t))
    for d, t in cases:
        assert accept_blocks(d, t, 4) == over.accept_blocks(d, t, 4)
        eos = [rng.randint(0, 3)]
        assert accept_blocks(d, t, 4, eos) == over.accept_blocks(d, t, 4, eos)
    assert accept_blocks([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 2, 9, 4], [5, 6, 7, 8]], 4) == \
        ([[1, 2, 9, 4]], [1, 2, 9], 2)


# Hand-worked acceptance (speculative_decode.py:895-953 with mrs.py:111-146
# greedy_match_verify, partial_block_fill = "draft_argmax"), each worked out
# by reading the reference loop, not by running either restatement:
#   (drafts, target argmax, eos ids) -> (committed, generated, accepted)
ACCEPT_HAND_CASES = [
    # rejection at position 1 with a tail that differs between draft and
    # target: the bonus is the target's 9, the block is filled from the
    # draft's own tail (3, 4), not the target's (8, 7)
    ([[1, 2, 3, 4]], [[1, 9, 8, 7]], None, ([[1, 9, 3, 4]], [1, 9], 1)),
    # K = 4, every block accepted: four whole blocks, no bonus token
    ([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]],
     [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]], None,
     ([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]],
      [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16], 16)),
    # rejection at the first position of the first block: one committed
    # block (the bonus then the draft's tail), later blocks never looked at
    ([[1, 2, 3, 4], [5, 6, 7, 8]], [[7, 6, 5, 4], [5, 6, 7, 8]], None, ([[7, 2, 3, 4]], [7], 0)),
    # block 0 accepted, block 1 rejected at its last position, block 2 dropped
    ([[1, 2, 3, 4], [5, 6, 7, 8], [9, 9, 9, 9]], [[1, 2, 3, 4], [5, 6, 7, 0], [9, 9, 9, 9]], None,
     ([[1, 2, 3, 4], [5, 6, 7, 0]], [1, 2, 3, 4, 5, 6, 7, 0], 7)),
    # an accepted block holding an EOS id ends the loop although block 1
    # would also be accepted
    ([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 2, 3, 4], [5, 6, 7, 8]], [3], ([[1, 2, 3, 4]], [1, 2, 3, 4], 4)),
    # the bonus itself is the EOS id: same block count as a plain rejection
    ([[1, 2, 3, 4], [5, 6, 7, 8]], [[1, 0, 3, 4], [5, 6, 7, 8]], [0], ([[1, 0, 3, 4]], [1, 0], 1)),
    # EOS ids that no generated token equals change nothing
    ([[1, 2, 0, 4], [5, 6, 7, 8]], [[1, 2, 0, 4], [5, 6, 7, 8]], [9],
     ([[1, 2, 0, 4], [5, 6, 7, 8]], [1, 2, 0, 4, 5, 6, 7, 8], 8)),
    # an EOS id in the draft's fill tail is committed but not generated
    ([[1, 2, 3, 0], [5, 6, 7, 8]], [[1, 9, 3, 0], [5, 6, 7, 8]], [0], ([[1, 9, 3, 0]], [1, 9], 1)),
]


@pytest.mark.parametrize("drafts,targets,eos,expect", ACCEPT_HAND_CASES)
def test_accept_blocks_hand_worked(drafts, targets, eos, expect):
    """Both the runner's acceptance and the oracle's restatement give the
    hand-worked result."""
    from oracle import verify as over
    from speculative.verify import accept_blocks
    assert accept_blocks(drafts, targets, 4, eos) == expect
    assert over.accept_blocks(drafts, targets, 4, eos) == expect


def test_empty_shapes_return_without_work():
    """M = 0 or N = 0: the workspace query says 0 bytes and the entry points
    return 0 before any launch (no device pointer is touched, so null
    pointers and a null stream are fine here)."""
    from kernels import _native
    lib = _native.lib()
    for M, N in ((0, 4096), (4, 0), (0, 0)):
        assert lib.simsd_thin_linear_workspace_bytes(M, N, 4096, 0, 0, 0, 0) == 0
        assert lib.simsd_rmsnorm_linear_workspace_bytes(M, N, 4096, 0, 0, 0, 0) == 0
        assert lib.simsd_thin_linear(None, 0, 0, None, 0, 0, None, 0, None, 0, 0, M, N, 4096, 0,
                                     0, 0, 0, 0, None, 0, None) == 0
        assert lib.simsd_thin_linear_noalloc(None, 0, 0, None, 0, 0, None, 0, None, 0, 0, M, N, 4096, 0,
                                             0, 0, 0, 0, None) == 0
    assert lib.simsd_thin_linear_noalloc(None, 0, 0, None, 0, 0, None, 0, None, 0, 0, 0, 4, 4, 7,
                                         0, 0, 0, 0, None) == -1       # bad dtype code
    assert b"dtype" in lib.simsd_last_error_string()
