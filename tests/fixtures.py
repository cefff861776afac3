"""Shared test helpers: golden-vector parsing and seeded synthetic inputs."""
from __future__ import annotations

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mlx-v0.32.0.oracle")


def unhex(s: str) -> bytes:
    return bytes.fromhex(s)


def parse_field(field: str):
    """'name:[shape]:dtype:hex' split from the right, as eredu-gguf/tests/oracle.rs:18-24."""
    prefix, dtype, data = field.rsplit(":", 2)
    return prefix, dtype, data


GOLDEN_IQ = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "llama-c0bc8591-iq.oracle")


def golden_iq_rows():
    """{ggml code: (raw block bytes, expected f16 bits)} of llama-c0bc8591-iq.oracle
    (eredu-gguf/tests/iquant.rs:113-127: two blocks per IQ type, llama.cpp's
    outputs rounded to f16, native byte order)."""
    rows = {}
    with open(GOLDEN_IQ) as f:
        for line in f:
            line = line.strip()
            if line:
                code, raw, expected = line.split("|")
                rows[int(code)] = (unhex(raw), np.frombuffer(unhex(expected), dtype="<u2").copy())
    return rows


def golden_rows():
    """{ggml code: dict(raw=bytes, weight=bytes, scales=bytes, biases=bytes, dequantized=bytes, block=int)}"""
    rows = {}
    with open(GOLDEN) as f:
        for line in f:
            line = line.strip()
            if not line:
                continue
            fields = line.split("|")
            code = int(fields[0])
            entry = {"raw": unhex(fields[1])}
            for field in fields[2:]:
                name, dtype, data = parse_field(field)
                key = name.split(".")[1].split(":")[0]
                entry[key] = unhex(data)
                entry[key + "_name"] = name
                entry[key + "_dtype"] = dtype
            rows[code] = entry
    return rows


# ------------------------------------------------------------ synthetic inputs

def f16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


# (block bytes, offsets of the f16 scale-like fields drawn |N(0, 0.01)|, offsets
# of the f16 offset fields drawn N(0, 0.01)) of the block types added after
# Q4_0 / Q8_0 / Q4_K (eredu-gguf/src/convert.rs:362-564).
KQUANT_HEADERS = {
    3: (20, (0,), (2,)),      # Q4_1: d, m
    6: (22, (0,), ()),        # Q5_0: d
    7: (24, (0,), (2,)),      # Q5_1: d, m
    10: (84, (80, 82), ()),   # Q2_K: d, dmin
    11: (110, (108,), ()),    # Q3_K: d
    13: (176, (0, 2), ()),    # Q5_K: d, dmin
    14: (210, (208,), ()),    # Q6_K: d
    20: (18, (0,), ()),       # IQ4_NL: d
    23: (136, (0,), ()),      # IQ4_XS: d (the u16 of high scale bits at 2 stays random)
}


def synthetic_blocks(ggml_type: int, nblocks: int, seed: int) -> np.ndarray:
    """GGML blocks with uniform random quant bytes and f16 d/dmin = f16(|N(0, 0.01)|)
    (the config-4 distribution; Q4_1 / Q5_1 offsets m = f16(N(0, 0.01)))."""
    rng = np.random.default_rng(seed)
    if ggml_type in KQUANT_HEADERS:
        nbytes, pos, signed = KQUANT_HEADERS[ggml_type]
        b = rng.integers(0, 256, size=(nblocks, nbytes), dtype=np.uint8)
        for off in pos + signed:
            v = rng.normal(0, 0.01, nblocks)
            b[:, off:off + 2] = f16_bits(v if off in signed else np.abs(v)).view(np.uint8).reshape(nblocks, 2)
        return np.ascontiguousarray(b.reshape(-1))
    if ggml_type == 2:  # Q4_0
        b = rng.integers(0, 256, size=(nblocks, 18), dtype=np.uint8)
        b[:, 0:2] = f16_bits(np.abs(rng.normal(0, 0.01, nblocks))).view(np.uint8).reshape(nblocks, 2)
    elif ggml_type == 8:  # Q8_0
        b = rng.integers(0, 256, size=(nblocks, 34), dtype=np.uint8)
        b[:, 0:2] = f16_bits(np.abs(rng.normal(0, 0.01, nblocks))).view(np.uint8).reshape(nblocks, 2)
    elif ggml_type == 12:  # Q4_K
        b = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
        b[:, 0:2] = f16_bits(np.abs(rng.normal(0, 0.01, nblocks))).view(np.uint8).reshape(nblocks, 2)
        b[:, 2:4] = f16_bits(np.abs(rng.normal(0, 0.01, nblocks))).view(np.uint8).reshape(nblocks, 2)
    else:
        raise ValueError(ggml_type)
    return np.ascontiguousarray(b.reshape(-1))


def synthetic_linear(N: int, K: int, group_size: int, bits: int, seed: int, scale_dtype: int = 2, std: float = 0.02):
    """W ~ N(0, std) quantized with the oracle's affine quantizer (input
    generator): returns (w u32 [N, K*bits/32], scales, biases)."""
    from oracle import oracle as orc

    W = normal_f32((N, K), seed) * np.float32(std)
    return orc.quantize_affine(W, group_size, bits, scale_dtype)


def normal_f32(shape, seed: int) -> np.ndarray:
    """Seeded N(0, 1) float32 samples; drawn on the GPU when one is present
    (host RNG is slow for the 58M-value full-size tensors)."""
    import torch

    if torch.cuda.is_available() and int(np.prod(shape)) > (1 << 20):
        g = torch.Generator(device="cuda").manual_seed(seed)
        return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).cpu().numpy()
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def synthetic_x(M: int, K: int, seed: int) -> np.ndarray:
    """bf16 bit patterns of x ~ N(0, 1)."""
    from oracle import oracle as orc

    return orc.f32_to_bf16_bits(normal_f32((M, K), seed))


# ------------------------------------------------------------ device transfer

def dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def dev_f16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.float16).cuda()


def dev_words(w: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(w, dtype=np.uint32).view(np.int32)).cuda()


def dev_u8(b: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint8)).cuda()


def dev_param(a: np.ndarray, dtype_code: int):
    """Scale/activation array of the given oracle dtype code onto the GPU."""
    import torch

    if dtype_code == 2:
        return dev_bf16(a)
    if dtype_code == 1:
        return dev_f16(a)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host_bits16(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_f32(t) -> np.ndarray:
    import torch

    if t.dtype == torch.bfloat16:
        return (host_bits16(t).astype(np.uint32) << 16).view(np.float32)
    return t.float().cpu().numpy()


def device_random_linear(N: int, K: int, group_size: int, bits: int, seed: int):
    """A packed projection drawn directly on the GPU (random codes; bf16 scales
    in [0.004, 0.008) and biases -s * (2^bits - 1) / 2, the magnitudes a
    N(0, 0.02) weight quantizes to) for shapes too large for the host
    quantizer: (w int32 [N, K*bits/32], scales, biases) device tensors."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randint(-(2**31), 2**31 - 1, (N, K * bits // 32), dtype=torch.int32, device="cuda", generator=g)
    s = (torch.rand((N, K // group_size), device="cuda", generator=g) * 0.004 + 0.004).to(torch.bfloat16)
    b = (-0.5 * ((1 << bits) - 1) * s.float()).to(torch.bfloat16)
    return w, s, b


def host_rows(w, s, b, rows):
    """Host copies (u32 words, bf16 bits) of the given output rows of a device projection."""
    import torch

    idx = torch.as_tensor(np.asarray(rows, dtype=np.int64), device=w.device)
    wr = w.index_select(0, idx).cpu().numpy().view(np.uint32)
    return wr, host_bits16(s.index_select(0, idx)), host_bits16(b.index_select(0, idx))
