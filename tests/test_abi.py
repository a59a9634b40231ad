"""C-ABI checks that need no GPU: the library loads, exports every entry point
that include/mamba_int.h declares, and rejects bad arguments before anything
is enqueued (no call here reaches the device)."""
import ctypes
import os
import re

import pytest

from conftest import REPO, PKG

HEADER = os.path.join(REPO, "include", "mamba_int.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:mi_status|const char \*|void)\s*(mi_\w+)\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert "mi_dyadic_scan" in names and "mi_bitlinear" in names and len(names) >= 18


def test_library_exports_every_declared_symbol():
    from mamba_int import _lib
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    bound = set(_lib.SIGNATURES) | {"mi_version", "mi_last_error_string", "mi_checkpoint_close"}
    assert set(declared()) == bound


def test_version_names_spec_and_arch():
    from mamba_int import _lib
    v = _lib.version()
    assert "mi-spec-2" in v and "gfx950" in v


def _fake(n=64):
    return ctypes.c_void_p(0x100000)  # never dereferenced: every call below fails validation


@pytest.mark.parametrize("call,status,needle", [
    (("mi_dyadic_scan", None, None, None, None, 15, None, None, None, 1, 4, 16, 0, None), 2, "nstate"),
    (("mi_dyadic_scan", None, None, None, None, 0, None, None, None, 1, 4, 16, 16, None), 4, "decay_shift"),
    (("mi_dyadic_scan", None, None, None, None, 15, None, None, None, 1, 4, 16, 16, None), 1, "required"),
    (("mi_ssd_chunked_scan", None, None, None, None, 15, None, None, None, None, 1, 8, 2, 16, 16, 0, None), 4, "chunk"),
    (("mi_bitlinear", None, 16, None, None, 16, 1, 4, 4, 17, 0, 0, 0, 0, None, ctypes.c_float(0), None, None), 2, "multiple of 16"),
    (("mi_bitlinear", None, 16, None, None, 16, 9, 4, 4, 16, 0, 0, 0, 0, None, ctypes.c_float(0), None, None), 4, "kind"),
    (("mi_bitlinear_gemv", "A16", 16, "W4", "O16", 16, 1, 100, 4, 16, 0, 0, 0, 0, None, ctypes.c_float(0), None, None), 2, "m <= 64"),
    (("mi_bitlinear", "A16", 8, "W4", "O16", 16, 1, 4, 4, 16, 0, 0, 0, 0, None, ctypes.c_float(0), None, None), 3, "lda"),
    (("mi_bitlinear", "A16", 16, "W4", "O16", 16, 4, 4, 4, 16, 0, 0, 0, 0, None, ctypes.c_float(0), None, None), 1, "x_scale"),
    (("mi_bitshift_norm", None, None, None, 4, 0, None, None), 2, "dim"),
    (("mi_conv_squareplus", None, 16, None, None, None, None, None, 1, 4, 18, None), 2, "multiple of 4"),
    (("mi_block_scan", None, None, None, 48, 16, None, 32, 16, None, 14, 13, None, None, None, 1, 4, 16, 16, None), 4, "decay_shift"),
    (("mi_norm_bitlinear", None, None, 1, None, None, None, 16, 1, 65, 16, 64, 0, None), 2, "m=65"),
    (("mi_norm_bitlinear", "A16", "A16", 0, "A16", "A16", "O16", 16, 1, 1, 16, 64, 0, None), 4, "stats_parts=0"),
    (("mi_norm_bitlinear", "A16", "W4", 2, "A16", "A16", "O16", 16, 1, 1, 16, 64, 0, None), 3, "row_stats"),
    (("mi_bitlinear_residual_parts", "A16", 64, "A16", "O16", 16, 65, 16, 64, 1, 0, 0, "A16", None), 2, "m=65"),
    (("mi_bitlinear_residual_parts", "A16", 32, "A16", "O16", 16, 1, 16, 32, 1, 0, 0, "A16", None), 2, "multiple of 64"),
    (("mi_bitlinear_residual_parts", "A16", 64, "A16", "O16", 16, 1, 16, 64, 1, 0, 0, None, None), 1, "stats_parts"),
    (("mi_bitlinear", "A16", 16, "W4", "O16", 16, 3, 4, 4, 16, 0, 1, 0, -1, None, ctypes.c_float(0), None, None), 4,
     "res_clamp"),
    (("mi_bitlinear_residual_parts", "A16", 64, "A16", "O16", 16, 1, 16, 64, 1, 0, -5, "A16", None), 4, "res_clamp"),
    (("mi_dt_scan_step", None, 80, 40, None, 2, None, None, 32, 16, None, 15, 13, None, None, 1, 16, 16, None), 2, "dt_rank"),
    (("mi_argmax_i32", None, 10, None, 1, 20, None), 2, "ld"),
    (("mi_bitshift_norm_parts", None, None, None, 4, 6, None, 1, 0, None), 2, "multiple of 4"),
    (("mi_bitshift_norm_parts", None, None, None, 70000, 8, None, 1, 0, None), 2, "65535"),
    (("mi_bitshift_norm_parts", None, None, None, 4, 8, None, 0, 0, None), 4, "nparts=0"),
    (("mi_bitshift_norm_parts", "A16", "A16", "A16", 4, 8, "W4", 2, 0, None), 3, "aligned"),
    (("mi_conv_step_xproj", None, 256, None, None, None, None, None, 5, 80, None, 80, 4, 100, None), 2, "multiple of 256"),
    (("mi_conv_step_xproj", None, 16384, None, None, None, None, None, 5, 80, None, 80, 4, 16384, None), 2, "<= 8192"),
    (("mi_conv_step_xproj", None, 512, None, None, None, None, None, 5, 300, None, 300, 4, 512, None), 2, "nx=300"),
    (("mi_conv_step_xproj", None, 512, None, None, None, None, None, 31, 80, None, 80, 4, 512, None), 4, "s_x=31"),
    (("mi_conv_step_xproj", None, 512, None, None, None, None, None, 5, 80, None, 80, 4, 512, None), 1, "required"),
    (("mi_conv_step_xpart", None, 512, None, None, None, None, None, 80, None, 4, 512, None), 2, "multiple of 1024"),
    (("mi_conv_step_xpart", None, 16384, None, None, None, None, None, 80, None, 4, 16384, None), 2, "<= 8192"),
    (("mi_conv_step_xpart", None, 1024, None, None, None, None, None, 300, None, 4, 1024, None), 2, "nx=300"),
    (("mi_conv_step_xpart", None, 1000, None, None, None, None, None, 80, None, 4, 1024, None), 2, "xz_stride=1000"),
    (("mi_conv_step_xpart", None, 1024, None, None, None, None, None, 80, None, 4, 1024, None), 1, "required"),
    (("mi_conv_step_xpart", None, 1024, None, None, None, None, None, 80, None, 70000, 1024, None), 2, "65535"),
    (("mi_dt_scan_step", None, 80, 48, None, 2, None, None, 3072, 1536, None, 15, 12, None, None, 70000, 1536, 16,
      None), 2, "65535"),
    (("mi_xpart_dt_scan_step", None, 96, 5, 48, None, 2, None, None, 3072, 1536, None, 15, 12, None, None, 70000,
      1536, 16, None), 2, "65535"),
    (("mi_conv_step_xpart", "A16", 1024, "W4", "A16", "A16", "A16", "A16", 80, "A16", 4, 1024, None), 3, "aligned"),
    (("mi_in_proj_conv", "A16", 64, "A16", 5, "A16", "A16", None, "A16", "A16", "O16", 208, 1, 4, 64, 100, None), 2,
     "multiple of 128"),
    (("mi_in_proj_conv", "A16", 32, "A16", 5, "A16", "A16", None, "A16", "A16", "O16", 256, 1, 4, 32, 128, None), 2,
     "multiple of 64"),
    (("mi_in_proj_conv", "A16", 64, "A16", 5, "A16", "A16", None, "A16", None, "O16", 256, 1, 4, 64, 128, None), 1,
     "required"),
    (("mi_in_proj_conv", "A16", 64, "A16", 5, "A16", "A16", "A16", "A16", "A16", "O16", 256, 1, 4, 64, 128, None), 4,
     "overlap"),
    (("mi_in_proj_conv", "A16", 64, "W4", 5, "A16", "A16", None, "A16", "A16", "O16", 256, 1, 4, 64, 128, None), 3,
     "16-byte"),
])
def test_argument_validation(call, status, needle):
    from mamba_int import _lib
    args = []
    for a in call[1:]:
        if a == "A16" or a == "O16":
            args.append(ctypes.c_void_p(0x100000))
        elif a == "W4":
            args.append(ctypes.c_void_p(0x100004))
        else:
            args.append(a)
    st = _lib.raw(call[0], *args)
    assert st == status, (_lib.last_error(), st)
    assert needle in _lib.last_error()


def test_zero_sizes_are_noops():
    from mamba_int import _lib
    assert _lib.raw("mi_dyadic_scan", None, None, None, None, 15, None, None, None, 0, 4, 16, 16, None) == 0
    assert _lib.raw("mi_bitlinear", None, 16, None, None, 16, 1, 0, 4, 16, 0, 0, 0, 0, None, ctypes.c_float(0), None,
                    None) == 0
    assert _lib.last_error() == ""


def test_ops_reject_host_tensors():
    import torch
    from mamba_int import ops
    with pytest.raises(ValueError):
        ops.bitshift_norm(torch.zeros(2, 16, dtype=torch.int32), torch.zeros(16, dtype=torch.int16))


def test_product_does_not_import_the_oracle():
    for root, _, files in os.walk(PKG):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(root, f)).read()
                assert not re.search(r"^\s*(import|from)\s+oracle", src, flags=re.M), f
                assert "liboracle" not in src, f


def test_decode_step_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors of mi_layer_params / mi_model_params have the C
    compiler's sizes and field offsets (a C program built from the header)."""
    import subprocess
    from mamba_int.native import CheckpointInfo, LayerParams, ModelParams
    src = tmp_path / "layout.c"
    lf = [f[0] for f in LayerParams._fields_]
    mf = [f[0] for f in ModelParams._fields_]
    cf = [f[0] for f in CheckpointInfo._fields_]
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"mamba_int.h\"\nint main(void){\n"
                   + 'printf("%zu\\n", sizeof(mi_layer_params));\n'
                   + "".join(f'printf("%zu\\n", offsetof(mi_layer_params, {f}));\n' for f in lf)
                   + 'printf("%zu\\n", sizeof(mi_model_params));\n'
                   + "".join(f'printf("%zu\\n", offsetof(mi_model_params, {f}));\n' for f in mf)
                   + 'printf("%zu\\n", sizeof(mi_checkpoint_info));\n'
                   + "".join(f'printf("%zu\\n", offsetof(mi_checkpoint_info, {f}));\n' for f in cf)
                   + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = ([ctypes.sizeof(LayerParams)] + [getattr(LayerParams, f).offset for f in lf]
            + [ctypes.sizeof(ModelParams)] + [getattr(ModelParams, f).offset for f in mf]
            + [ctypes.sizeof(CheckpointInfo)] + [getattr(CheckpointInfo, f).offset for f in cf])
    assert got == want


def test_decode_step_validation():
    """mi_decode_step / mi_decode_workspace_size reject bad models before enqueueing."""
    from mamba_int import _lib
    from mamba_int.native import ModelParams
    p = ModelParams(768, 24, 32000, 16, 48, None, None, None, None)
    pp = ctypes.cast(ctypes.pointer(p), ctypes.c_void_p)
    n = ctypes.c_size_t(0)
    np_ = ctypes.cast(ctypes.pointer(n), ctypes.c_void_p)
    assert _lib.raw("mi_decode_workspace_size", None, 8, np_) == 1
    assert _lib.raw("mi_decode_workspace_size", pp, 8, np_) == 1 and "required" in _lib.last_error()
    p.emb = p.gamma_f = p.w_head = 0x1000
    p.layers = ctypes.cast(ctypes.c_void_p(0x1000), type(p.layers))
    assert _lib.raw("mi_decode_workspace_size", pp, 65, np_) == 2 and "m=65" in _lib.last_error()
    p.d_model = 800
    assert _lib.raw("mi_decode_workspace_size", pp, 8, np_) == 2 and "d_model" in _lib.last_error()
    p.d_model = 768
    assert _lib.raw("mi_decode_workspace_size", pp, 8, np_) == 0 and n.value > 0
    ws = n.value
    args = (pp, 8, None, None, None, 0, None, None, None, ctypes.c_size_t(ws), None)
    assert _lib.raw("mi_decode_step", *args) == 1 and "required" in _lib.last_error()
