"""The C-ABI boundary on the CPU: the library loads, exports every entry point
declared in include/eredu_hip.h, and rejects bad arguments with a status and
a thread-local message before anything is launched (no compute here)."""
import ctypes
import os
import re
import subprocess
import threading

import pytest

from eredu_amd import _native
from eredu_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "eredu_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    assert declared_functions() == sorted(
        ["eq_last_error", "eq_version", "eq_quantized_matmul", "eq_quantized_matmul_batched", "eq_dequantize",
         "eq_gguf_convert_affine", "eq_gguf_dequantize", "eq_rms_norm", "eq_rope_attention_decode", "eq_silu_mul",
         "eq_embedding", "eq_argmax", "eq_quantized_matmul_batched_prologue", "eq_quantize",
         "eq_gguf_linear", "eq_gather_qmm", "eq_rope_attention_decode_noalloc", "eq_gguf_convert_mxfp4",
         "eq_gguf_embedding", "eq_gguf_grouped_linear", "eq_rope_attention_decode_at", "eq_advance_position",
         "eq_quantized_matmul_swiglu"]
    )


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "build the library first (python -m eredu_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (eq_[a-z0-9_]+)", out))
    for name in declared_functions():
        assert name in exported, name
    # and the ctypes table covers them all
    assert set(_native.SIGNATURES) == set(declared_functions())


def test_header_compiles_as_c():
    src = f'#include "{HEADER}"\nint (*f)(void) = eq_version;\nint main(void) {{ return f != 0; }}\n'
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-x", "c", "-fsyntax-only", "-"],
                         input=src, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


L = _native.lib()


def call_qmm(**kw):
    args = dict(y=1, x=1, w=1, s=1, b=None, M=1, N=16, K=64, transpose=True, gs=64, bits=4, mode=b"affine",
                xd=2, sd=2)
    args.update(kw)
    return L.eq_quantized_matmul(args["y"], args["x"], args["w"], args["s"], args["b"], args["M"], args["N"],
                                 args["K"], args["transpose"], args["gs"], args["bits"], args["mode"], args["xd"],
                                 args["sd"], None)


@pytest.mark.parametrize(
    "kw,needle",
    [
        (dict(gs=48), "group_size must be 16 or a positive multiple of 32"),
        (dict(bits=7), "bits must be one of 2, 3, 4, 5, 6 or 8"),
        (dict(bits=3, gs=16, K=16), "does not fill whole 32-bit words"),
        (dict(bits=5, gs=16, transpose=False, N=16), "does not fill whole 32-bit words"),
        (dict(K=96), "not divisible by group_size"),
        (dict(transpose=False, N=40), "not divisible by group_size"),
        (dict(mode=b"mxfp4"), "MXFP4 requires group_size=32 and bits=4"),
        (dict(mode=b"mxfp4", gs=32, sd=2), "E8M0 bytes"),
        (dict(mode=b"nf4"), "invalid quantization mode"),
        (dict(xd=7), "invalid dtype"),
        (dict(N=0), "invalid shape"),
        (dict(y=None), "null pointer"),
    ],
)
def test_quantized_matmul_rejects(kw, needle):
    assert call_qmm(**kw) != 0
    assert needle in L.eq_last_error().decode()


def test_zero_rows_is_a_no_op():
    assert call_qmm(M=0, y=None, x=None) != 0  # null pointers are still rejected
    assert call_qmm(M=0) == 0
    assert L.eq_last_error().decode() == ""


def test_error_message_is_thread_local():
    assert call_qmm(gs=48) != 0
    seen = {}

    def other():
        seen["before"] = L.eq_last_error().decode()
        call_qmm(bits=7)
        seen["after"] = L.eq_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == ""
    assert "bits" in seen["after"]
    assert "group_size" in L.eq_last_error().decode()


@pytest.mark.parametrize(
    "args,needle",
    [
        (dict(ty=16), "unsupported GGML tensor type"),
        (dict(ty=39), "unsupported GGML tensor type"),
        (dict(cols=48), "not divisible by group size 32"),
        (dict(cols=264, ty=14), "not divisible by group size 16"),
        (dict(ty=20), "no affine conversion"),
        (dict(cols=288, ty=12), "not divisible by block length 256"),
        (dict(raw_len=17), "payload length does not match descriptor"),
        (dict(endian=5), "invalid endian"),
    ],
)
def test_gguf_convert_rejects(args, needle):
    a = dict(ty=2, rows=2, cols=64, raw_len=None, endian=0)
    a.update(args)
    if a["raw_len"] is None:
        vals, nbytes = {2: (32, 18), 8: (32, 34), 12: (256, 144)}.get(a["ty"], (32, 18))
        a["raw_len"] = a["rows"] * a["cols"] // vals * nbytes
    buf = ctypes.create_string_buffer(64)
    ptr = ctypes.cast(buf, ctypes.c_void_p)
    rc = L.eq_gguf_convert_affine(ptr, ptr, ptr, ptr, a["raw_len"], a["ty"], a["rows"], a["cols"], a["endian"], None)
    assert rc != 0
    assert needle in L.eq_last_error().decode()


def test_gguf_convert_mxfp4_rejects():
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    _rejects(L.eq_gguf_convert_mxfp4(p, p, p, 17, 1, 48, None), "not divisible by 32")
    _rejects(L.eq_gguf_convert_mxfp4(p, p, p, 18, 1, 32, None), "payload length")
    _rejects(L.eq_gguf_convert_mxfp4(None, p, p, 17, 1, 32, None), "null")
    assert L.eq_gguf_convert_mxfp4(None, None, None, 0, 0, 32, None) == 0  # nothing to convert


def test_gguf_dequant_rejects_bad_definition_and_dtype():
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.cast(buf, ctypes.c_void_p)
    aligned = (p.value + 15) // 16 * 16
    assert L.eq_gguf_dequantize(aligned, aligned, 36, 2, 2, 32, 0, 9, 2, None) != 0
    assert "definition" in L.eq_last_error().decode()
    assert L.eq_gguf_dequantize(aligned, aligned, 36, 2, 2, 32, 0, 0, 1, None) != 0
    assert "bf16 or f32" in L.eq_last_error().decode()


def test_gguf_embedding_rejects():
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.cast(buf, ctypes.c_void_p)
    a = (p.value + 15) // 16 * 16
    f32, bf16 = 0, 2
    _rejects(L.eq_gguf_embedding(a, a, 144, 12, 1, 256, a, 1, 0, 1, None), "bf16 or f32")
    _rejects(L.eq_gguf_embedding(a, a, 144, 12, 1, 256, a, -1, 0, f32, None), "token count")
    _rejects(L.eq_gguf_embedding(None, a, 144, 12, 1, 256, a, 1, 0, f32, None), "non-null")
    _rejects(L.eq_gguf_embedding(a, a, 144, 12, 1, 256, None, 1, 0, bf16, None), "non-null")
    _rejects(L.eq_gguf_embedding(a + 8, a, 144, 12, 1, 256, a, 1, 0, f32, None), "aligned")
    _rejects(L.eq_gguf_embedding(a, a, 143, 12, 1, 256, a, 1, 0, f32, None), "")  # payload length
    assert L.eq_gguf_embedding(None, a, 144, 12, 1, 256, None, 0, 0, f32, None) == 0  # no tokens


def test_gguf_grouped_linear_rejects():
    buf = ctypes.create_string_buffer(8192)
    p = ctypes.cast(buf, ctypes.c_void_p)
    a = (p.value + 15) // 16 * 16
    bf16 = _native.EQ_DTYPE_BF16
    # 2 experts x 8 rows x 256 Q8_0 values: 2 * 8 * 8 * 34 bytes
    nraw = 2 * 8 * 8 * 34
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 2, 2, 8, 256, a, 1, 0, bf16, True, None), "covers Q4_K")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 8, 0, 8, 256, a, 1, 0, bf16, True, None), "bank shape")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw - 1, 8, 2, 8, 256, a, 1, 0, bf16, True, None), "")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 8, 2, 8, 256, a, 1, 0, 1, True, None), "bf16 activations")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 8, 2, 8, 256, a, -1, 0, bf16, True, None), "route count")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 8, 2, 8, 256, None, 1, 0, bf16, True, None), "null")
    _rejects(L.eq_gguf_grouped_linear(a, a + 2, a, nraw, 8, 2, 8, 256, a, 1, 0, bf16, True, None), "aligned")
    _rejects(L.eq_gguf_grouped_linear(a, a, a, nraw, 8, 2, 8, 256, a, 17, 0, bf16, True, None), "N % 128")
    assert L.eq_gguf_grouped_linear(None, None, a, nraw, 8, 2, 8, 256, None, 0, 0, bf16, True, None) == 0


def test_host_mirror_fails_loudly_without_gpu_tensors():
    import torch

    from eredu_amd import EreduError, quantized_matmul

    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    w = torch.zeros(16, 8, dtype=torch.int32)
    s = torch.zeros(16, 1, dtype=torch.bfloat16)
    with pytest.raises(EreduError, match="GPU"):
        quantized_matmul(x, w, s, s, transpose=True)


def _rejects(status, fragment):
    assert status == 1
    assert fragment in L.eq_last_error().decode()


def test_decode_ops_reject_bad_arguments():
    bf16, f32 = _native.EQ_DTYPE_BF16, _native.EQ_DTYPE_F32
    # rms_norm: dtype, dim, alignment, null
    _rejects(L.eq_rms_norm(16, 16, None, 16, 1, 4096, 1e-5, f32, None), "only bf16")
    _rejects(L.eq_rms_norm(16, 16, None, 16, 1, 4095, 1e-5, bf16, None), "multiple of 8")
    _rejects(L.eq_rms_norm(16, 18, None, 16, 1, 4096, 1e-5, bf16, None), "aligned")
    _rejects(L.eq_rms_norm(None, 16, None, 16, 1, 4096, 1e-5, bf16, None), "null")
    _rejects(L.eq_rms_norm(16, 16, None, 16, 1, 4096, -1.0, bf16, None), "eps")
    # attention: head width, grouping, position range
    att = lambda **k: L.eq_rope_attention_decode(16, 16, 16, 16, 16, 16, 16, k.get("pos", 10), k.get("max_seq", 64),
                                                  k.get("h", 32), k.get("kv", 8), k.get("d", 128), 0.088,
                                                  k.get("dt", bf16), None)
    _rejects(att(d=64), "head_dim")
    _rejects(att(h=33), "n_heads")
    _rejects(att(h=64, kv=8), "n_heads")
    _rejects(att(pos=64), "pos")
    _rejects(att(pos=-1), "pos")
    _rejects(att(dt=f32), "only bf16")
    # attention at a device position: the same shape rules, the position pointer, max_seq
    att_at = lambda **k: L.eq_rope_attention_decode_at(16, 16, 16, 16, 16, 16, 16, k.get("pos", 16),
                                                        k.get("max_seq", 64), k.get("h", 32), k.get("kv", 8),
                                                        k.get("d", 128), 0.088, k.get("dt", bf16), None)
    _rejects(att_at(d=64), "head_dim")
    _rejects(att_at(h=64, kv=8), "n_heads")
    _rejects(att_at(pos=None), "null")
    _rejects(att_at(max_seq=0), "max_seq")
    _rejects(att_at(max_seq=131073), "131072")
    _rejects(att_at(dt=f32), "only bf16")
    _rejects(L.eq_advance_position(None, None), "null")
    # gate/up with the SwiGLU epilogue: shape, layout and prologue rules, before any launch
    import ctypes
    from eredu_amd import _native as n
    sw = lambda pro=None, **k: L.eq_quantized_matmul_swiglu(
        k.get("out", 1 << 20), 16, 16, 1 << 21, None, k.get("F", 512), k.get("K", 4096), k.get("gs", 64),
        k.get("bits", 4), b"affine", k.get("xdt", bf16), bf16, ctypes.byref(pro) if pro is not None else None, None)
    _rejects(sw(F=500), "multiple of 8")
    _rejects(sw(K=100), "multiple of 64")
    _rejects(sw(gs=32), "group size 64")
    _rejects(sw(bits=3), "4- or 8-bit")
    _rejects(sw(xdt=f32), "bf16")
    _rejects(sw(out=None), "null")
    _rejects(sw(n.ActivationPrologue(n.EQ_PROLOGUE_SILU_MUL, 16, None, None, 0.0)), "RMS_NORM")
    _rejects(sw(n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, None, 16, None, 1e-5), K=8192), "4096")
    _rejects(sw(n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, None, 16, None, -1.0)), "eps")
    # the output overlapping the packed codes
    _rejects(sw(out=64), "overlaps")
    # silu_mul, embedding, argmax
    _rejects(L.eq_silu_mul(16, 16, 16, 12, bf16, None), "multiple of 8")
    _rejects(L.eq_embedding(16, 16, 16, 70000, 100, 64, bf16, None), "n_tokens")
    _rejects(L.eq_embedding(16, 16, 16, 1, 100, 60, bf16, None), "dim")
    _rejects(L.eq_argmax(16, 16, 1, 0, bf16, None), "0 < n")
    # zero-size calls succeed without launching
    assert L.eq_rms_norm(16, 16, None, 16, 0, 4096, 1e-5, bf16, None) == 0
    assert L.eq_silu_mul(16, 16, 16, 0, bf16, None) == 0


def test_quantize_rejects_bad_arguments():
    bf16 = _native.EQ_DTYPE_BF16
    _rejects(L.eq_quantize(16, 16, 16, 16, 4, 100, 64, 4, b"affine", bf16, None), "multiple of group_size")
    _rejects(L.eq_quantize(16, 16, 16, 16, 4, 128, 48, 4, b"affine", bf16, None), "group")
    _rejects(L.eq_quantize(16, 16, 16, 16, 4, 128, 64, 7, b"affine", bf16, None), "bits")
    _rejects(L.eq_quantize(16, 16, 16, 16, 4, 16, 16, 3, b"affine", bf16, None), "whole 32-bit words")
    _rejects(L.eq_quantize(16, 16, 16, 16, 4, 128, 64, 4, b"affine", 9, None), "dtype")
    _rejects(L.eq_quantize(None, 16, 16, 16, 4, 128, 64, 4, b"affine", bf16, None), "null")
    assert L.eq_quantize(16, 16, 16, 16, 0, 128, 64, 4, b"affine", bf16, None) == 0


def test_gguf_linear_rejects_bad_arguments():
    bf16 = _native.EQ_DTYPE_BF16
    # Q4_0 is not a native-linear type; payload length must match; bf16 only
    _rejects(L.eq_gguf_linear(16, 16, 16, 18 * 8, 2, 1, 2, 128, 0, bf16, None), "Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS")
    _rejects(L.eq_gguf_linear(16, 16, 16, 84 * 2, 10, 1, 2, 256, 0, bf16, None), "Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS")
    _rejects(L.eq_gguf_linear(16, 16, 16, 100, 12, 1, 2, 256, 0, bf16, None), "payload length")
    _rejects(L.eq_gguf_linear(16, 16, 16, 2 * 144, 12, 1, 2, 256, 0, _native.EQ_DTYPE_F32, None), "bf16")
    _rejects(L.eq_gguf_linear(16, 18, 16, 2 * 144, 12, 1, 2, 256, 0, bf16, None), "aligned")
    assert L.eq_gguf_linear(16, 16, 16, 2 * 144, 12, 0, 2, 256, 0, bf16, None) == 0


def test_gather_qmm_rejects_bad_arguments():
    bf16 = _native.EQ_DTYPE_BF16
    # (y, x, w, scales, biases, lhs, rhs, batch, x_batches, w_batches, M, N, K, transpose, gs, bits, mode,
    #  x_dtype, scale_dtype, sorted, stream)
    args = [16, 16, 16, 16, None, 16, 16, 4, 4, 8, 1, 32, 128, True, 64, 4, b"affine", bf16, bf16, False, None]

    def call(**kw):
        a = list(args)
        names = ["y", "x", "w", "s", "b", "lhs", "rhs", "batch", "xb", "wb", "M", "N", "K", "t", "gs", "bits",
                 "mode", "xd", "sd", "sorted", "st"]
        for k, v in kw.items():
            a[names.index(k)] = v
        return L.eq_gather_qmm(*a)

    _rejects(call(gs=48), "group_size")
    _rejects(call(bits=7), "bits")
    _rejects(call(bits=3, gs=16, K=16), "whole 32-bit words")
    _rejects(call(mode=b"mxfp4"), "MXFP4 requires group_size=32 and bits=4")
    _rejects(call(mode=b"mxfp4", gs=32, sd=3, b=16), "no biases")
    _rejects(call(xd=7), "dtype")
    _rejects(call(K=96), "divisible")
    _rejects(call(wb=0), "w_batches")
    _rejects(call(lhs=None, xb=3), "lhs_indices")     # 3 x batches for 4 outputs, no indices
    _rejects(call(rhs=None, wb=8), "rhs_indices")
    _rejects(call(w=None), "null")
    _rejects(call(t=False, N=128, M=8 * 65535 + 1), "rows per batch")
    assert call(batch=0) == 0 and call(M=0) == 0      # nothing to do, nothing launched
