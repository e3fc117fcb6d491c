"""C-ABI library checks that need no GPU: it loads, exports every symbol the header
declares, sizes its workspace sensibly and rejects bad arguments before touching
the device.  The Python entry point's argument checks run on CPU tensors too."""
import ctypes
import os
import re

import pytest
import torch

from conftest import REPO, pkg

HEADER = os.path.join(REPO, "include", "moe_mi355.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"MOE_MI355_API\s+[\w\s\*]+?\b(moe_mi355_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return pkg("kernel")._build_extension()


def test_header_declares_entry_points():
    syms = header_symbols()
    for s in ("moe_mi355_forward", "moe_mi355_route", "moe_mi355_dispatch",
              "moe_mi355_workspace_bytes", "moe_mi355_strerror"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    for s in header_symbols():
        assert hasattr(lib, s), s


def test_exported_symbols_are_only_the_c_abi():
    path = pkg("kernel").library_path()
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(header_symbols())


def test_workspace_bytes(lib):
    k = pkg("kernel")
    sizes = [k.workspace_bytes(t) for t in (0, 1, 8, 64, 1024, 8192)]
    assert all(s % 256 == 0 for s in sizes)
    assert sizes == sorted(sizes)
    lay = k.workspace_layout(64)
    assert lay.total == sizes[3]
    offs = [lay.topk_ids, lay.topk_weights, lay.inverse_rows, lay.meta, lay.tiles,
            lay.sorted_tokens, lay.sorted_weights, lay.chunk_counts, lay.token_masks, lay.row_scales,
            lay.intermediate, lay.expert_out, lay.expert_out_exp]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert lay.token_masks + 64 * 4 <= lay.row_scales                        # [T] uint32
    assert lay.row_scales + 56 * 64 * 8 * 4 <= lay.intermediate               # [56, 8T] fp32
    assert lay.intermediate + 64 * 8 * (2048 * 4 + 128) <= lay.intermediate_scales  # hi/lo, fp16, exps
    assert lay.expert_out + 64 * 8 * 7168 * 2 <= lay.expert_out_exp          # fp16 expert rows
    assert lay.expert_out_exp + 64 * 8 * 448 <= lay.total                    # their group exponents
    assert lay.max_tiles == (64 * 8 + 15) // 16 + 32   # sized for the smallest tile height
    assert lib.moe_mi355_workspace_bytes(-1) == 0
    assert lib.moe_mi355_workspace_bytes(1 << 21) == 0
    # no full-size shadow copies for values beyond the fp16 range: about 23 KB per routed
    # row; with fp32 copies of the expert rows and bf16 copies of C it was 3.56 GB at
    # T = 8192, and the cut must be at least 40 %
    assert k.workspace_bytes(8192) < 8192 * 8 * 23.5e3
    assert k.workspace_bytes(8192) <= 0.6 * 3_556_769_792


def test_forward_rejects_bad_arguments_without_a_gpu(lib):
    k = pkg("kernel")
    a = k.MoeArgs()
    assert lib.moe_mi355_forward(None, None) == -1
    a.T = -3
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -2
    a.T = 0
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == 0   # nothing to do
    a.T = 4
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -1  # NULL tensors
    fake = 1 << 20
    for f in ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
              "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
              "output"):
        setattr(a, f, fake)
    a.hidden_states = fake + 8
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -4  # misaligned
    a.hidden_states = fake
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -3  # no workspace
    a.workspace = fake
    a.workspace_bytes = 100
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -3  # too small
    assert lib.moe_mi355_dispatch(None, None, 4, 0, 48, None, None, None, None, None, None, None, None) == -6
    assert lib.moe_mi355_route(None, None, -1, 1.0, None, None, None) == -2
    assert lib.moe_mi355_strerror(-3).decode().startswith("workspace")
    assert lib.moe_mi355_debug_e4m3_to_bf16(None, None, 4, None) == -1


def _cpu_args(T=4):
    return [torch.zeros(T, 256), torch.zeros(256, dtype=torch.bfloat16),
            torch.zeros(T, 7168, dtype=torch.float8_e4m3fn), torch.ones(56, T),
            torch.zeros(32, 4096, 7168, dtype=torch.float8_e4m3fn), torch.ones(32, 32, 56),
            torch.zeros(32, 7168, 2048, dtype=torch.float8_e4m3fn), torch.ones(32, 56, 16),
            0, 2.5, torch.zeros(T, 7168, dtype=torch.bfloat16)]


@pytest.fixture(scope="module")
def cpu_args():
    return _cpu_args()


@pytest.mark.parametrize("idx,bad,msg", [
    (0, torch.zeros(4, 256, dtype=torch.float16), "routing_logits must have dtype"),
    (1, torch.zeros(256), "routing_bias must have dtype"),
    (1, torch.zeros(128, dtype=torch.bfloat16), "routing_bias must have shape"),
    (2, torch.zeros(4, 7168, dtype=torch.bfloat16), "hidden_states must have dtype"),
    (3, torch.ones(4, 56), "hidden_states_scale must have shape"),
    (5, torch.ones(32, 56, 32), "gemm1_weights_scale must have shape"),
    (7, torch.ones(32, 16, 56), "gemm2_weights_scale must have shape"),
    (10, torch.zeros(4, 7168), "output must have dtype"),
    (10, torch.zeros(3, 7168, dtype=torch.bfloat16), "output must have shape"),
])
def test_kernel_validates_like_the_reference(cpu_args, idx, bad, msg):
    k = pkg("kernel")
    args = list(cpu_args)
    args[idx] = bad
    with pytest.raises(ValueError, match=msg):
        k.kernel(*args)


def test_kernel_rejects_host_tensors(cpu_args):
    k = pkg("kernel")
    with pytest.raises(ValueError, match="GPU tensor"):
        k.kernel(*cpu_args)


def test_kernel_signature_matches_reference():
    """Exactly the reference's 11 parameters, same names and order
    (solution/python/kernel.py:95-107): the harness's builder checks the DPS
    parameter count and rejects variadic arguments (README.md:227-257)."""
    import inspect
    k = pkg("kernel")
    params = list(inspect.signature(k.kernel).parameters.values())
    assert all(p.kind == p.POSITIONAL_OR_KEYWORD and p.default is p.empty for p in params)
    assert [p.name for p in params] == [
        "routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
        "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
        "local_expert_offset", "routed_scaling_factor", "output"]


def test_config_toml_names_the_entry_point():
    import tomli
    with open(os.path.join(REPO, "flash-infer-bench-starter-kit_amd", "config.toml"), "rb") as f:
        cfg = tomli.load(f)
    assert cfg["solution"]["definition"] == "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
    assert cfg["build"]["entry_point"] == "kernel.py::kernel"
    assert cfg["build"]["destination_passing_style"] is True


def test_no_oracle_import_in_product():
    pkg_dir = os.path.join(REPO, "flash-infer-bench-starter-kit_amd")
    for root, _, files in os.walk(pkg_dir):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, f)).read()
                assert "moe_oracle" not in text and "oracle/" not in text, f


def _fake_args(k, T=4):
    """Arguments whose pointers are aligned but point nowhere: only calls that the
    library rejects before any launch may use them."""
    a = k.MoeArgs()
    fake = 1 << 20
    for f in ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
              "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
              "output", "workspace"):
        setattr(a, f, fake)
    a.T = T
    a.workspace_bytes = k.workspace_bytes(T)
    return a


@pytest.mark.parametrize("g1,g2", [(4, 1), (3, 3), (1, 4), (2, 2), (0, 1), (5, 5), (3, 5), (3, 4), (4, 4),
                                   (1, 2), (5, 2), (2, 6), (7, 3), (7, 1), (9, 5), (8, 1), (8, 3)])
def test_forced_plan_that_cannot_run_is_an_error(lib, g1, g2):
    """A GEMM pair that cannot run together (GEMM1 writes hi/lo C but GEMM2 reads fp16,
    mismatched tile heights, GEMM1 9 with any GEMM2 but 6, unknown variants: GEMM1 3,
    GEMM2 2 and 4, kernels of earlier builds that no plan used, are gone) is rejected
    before any launch with
    MOE_ERR_BAD_FLAGS, and the Python entry turns the status into a RuntimeError."""
    k = pkg("kernel")
    a = _fake_args(k)
    a.flags = k.plan_flags(g1, g2)
    rc = lib.moe_mi355_forward(ctypes.byref(a), None)
    assert rc == -7
    assert "forced kernel plan" in lib.moe_mi355_strerror(rc).decode()
    with pytest.raises(RuntimeError, match="moe_mi355_forward failed: unknown flag bits"):
        k._check(rc, "moe_mi355_forward")
    lay = k.WorkspaceLayout()
    assert lib.moe_mi355_get_workspace_layout(4, a.flags, ctypes.byref(lay)) == -7


@pytest.mark.parametrize("flags", [1 << 20, 1 << 9, 4 | 8, 1 << 31, 1 << 5])
def test_unknown_flag_bits_are_an_error(lib, flags):
    """Unknown bits, variant bits without the force bit, and both token-scale forms at
    once are rejected."""
    k = pkg("kernel")
    a = _fake_args(k)
    a.flags = flags - (1 << 32) if flags >= 1 << 31 else flags
    assert lib.moe_mi355_forward(ctypes.byref(a), None) == -7


def test_list_order_flag_is_known_and_keeps_the_plan():
    """FLAG_LIST_ORDER (16) only changes which workgroup takes a prefill GEMM1 item: it is
    accepted alone and with a forced plan, and the layout is the same as without it."""
    k = pkg("kernel")
    assert k.FLAG_LIST_ORDER == 16
    for T, base in ((2000, 0), (700, k.plan_flags(4, 5)), (64, 0)):
        a, b = k.workspace_layout(T, base), k.workspace_layout(T, base | k.FLAG_LIST_ORDER)
        assert (a.total, a.tile_m, a.intermediate_format) == (b.total, b.tile_m, b.intermediate_format)


def test_layout_reports_the_forced_plan():
    k = pkg("kernel")
    assert k.workspace_layout(64).tile_m == 16 and k.workspace_layout(64).intermediate_format == 0
    # 32-row streaming tiles up to T = 199, then the token-sharing GEMM1 on 64-row tiles
    # (fp16 C for the token-sharing GEMM2 up to T = 559, C converted to the hi/lo form for
    # the prefill GEMM2 beyond), then 256-row prefill tiles
    assert [k.workspace_layout(t).tile_m for t in (89, 199, 200, 559, 560, 1344, 1345)] == \
        [32, 32, 64, 64, 64, 64, 256]
    assert [k.workspace_layout(t).intermediate_format for t in (199, 200, 559, 560, 1344, 1345)] == \
        [0, 0, 0, 2, 2, 1]
    # GEMM1 computes the dispatch itself up to T = 64, a dispatch launch from T = 65
    assert [k.workspace_layout(t).dispatch_in_gemm1 for t in (1, 8, 64, 65, 200, 9000)] == [1, 1, 1, 0, 0, 0]
    assert k.workspace_layout(64, k.plan_flags(1, 1)).dispatch_in_gemm1 == 0
    assert k.workspace_layout(8, k.plan_flags(5, 1)).dispatch_in_gemm1 == 1
    lay = k.WorkspaceLayout()
    lib = k._build_extension()
    assert lib.moe_mi355_get_workspace_layout(65, k.plan_flags(5, 1), ctypes.byref(lay)) == -7
    assert lib.moe_mi355_get_workspace_layout(8, k.plan_flags(5, 3), ctypes.byref(lay)) == -7
    # GEMM2 writes the output itself (variant 6) by default up to T = 22, when forced up to
    # T = 32, after GEMM1 variant 9, 5 or 1
    assert [k.workspace_layout(t).combine_in_gemm2 for t in (1, 8, 22, 23, 32, 33, 64, 200)] == \
        [1, 1, 1, 0, 0, 0, 0, 0]
    assert k.workspace_layout(32, k.plan_flags(5, 6)).combine_in_gemm2 == 1
    assert k.workspace_layout(8, k.plan_flags(5, 1)).combine_in_gemm2 == 0
    assert k.workspace_layout(8, k.plan_flags(1, 6)).combine_in_gemm2 == 1
    assert k.workspace_layout(8, k.plan_flags(1, 6)).dispatch_in_gemm1 == 0
    for t, g1 in ((33, 5), (8, 2), (8, 4), (8, 7)):
        assert lib.moe_mi355_get_workspace_layout(t, k.plan_flags(g1, 6), ctypes.byref(lay)) == -7
    # GEMM1 variant 9 (routing, dispatch and GEMM1 in one launch) up to T = 8, with GEMM2
    # variant 6 only
    for t in (4, 5, 8):
        assert k.workspace_layout(t, k.plan_flags(9, 6)).dispatch_in_gemm1 == 1
        assert k.workspace_layout(t, k.plan_flags(9, 6)).combine_in_gemm2 == 1
        assert k.workspace_layout(t, k.plan_flags(9, 6)).tile_m == 16
    for t, g2 in ((9, 6), (16, 6), (4, 1), (4, 3), (4, 5), (1, 1)):
        assert lib.moe_mi355_get_workspace_layout(t, k.plan_flags(9, g2), ctypes.byref(lay)) == -7
    assert lib.moe_mi355_get_workspace_layout(4, k.plan_flags(9, 6) | k.FLAG_ROW_SCALES_ON,
                                              ctypes.byref(lay)) == -7
    # the token-sharing GEMM2 (variant 7) reads the fp16 C of the token-sharing GEMM1s on
    # their 64-row tiles: no conversion, no second tile list
    lay7 = k.workspace_layout(600, k.plan_flags(8, 7))
    assert (lay7.tile_m, lay7.intermediate_format) == (64, 0)
    for g1 in (1, 2, 4, 5, 9):
        assert lib.moe_mi355_get_workspace_layout(600, k.plan_flags(g1, 7), ctypes.byref(lay)) == -7
    # gathered token scales need the separate dispatch
    assert k.workspace_layout(8, k.FLAG_ROW_SCALES_ON).dispatch_in_gemm1 == 0
    assert k.workspace_layout(8, k.FLAG_ROW_SCALES_OFF).dispatch_in_gemm1 == 1
    assert lib.moe_mi355_get_workspace_layout(8, k.plan_flags(5, 1) | k.FLAG_ROW_SCALES_ON,
                                              ctypes.byref(lay)) == -7


def test_environment_does_not_change_the_plan():
    """The library reads no environment: variables that older builds read for plan
    overrides leave the plan alone."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); from conftest import pkg; "
            "k = pkg('kernel'); l = k.workspace_layout(64); print(l.tile_m, l.intermediate_format)"
            % os.path.join(REPO, "tests"))
    env = dict(os.environ, MOE_MI355_G1="4", MOE_MI355_G2="5", MOE_MI355_ROW_SCALES="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         cwd=os.path.join(REPO, "tests"), timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["16", "0"]
