"""Regenerate the golden fixtures in this folder.

The reference repository holds no golden vectors (its inputs are unseeded torch.randn). Its tests
check the kernels against torch's CPU scaled_dot_product_attention on fp32 copies
(test_flash_atten.py:459-461, 498-499) and CPU torch.matmul (test_mma.py:260-261). These fixtures
are computed with that same oracle path, in float64, on inputs from the portable seeded generator
(oracle.portable_normal / portable_uniform, rounded to the kernel dtype), so the inputs are not
stored: only a checksum of them and the expected outputs.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

# name: (seed, B, H, Hkv, M, N, D, dtype, causal, input_scale)
ATTENTION_CASES = {
    "cfg1_b1h4n512d64_f16": (20260328, 1, 4, 4, 512, 512, 64, oracle.DTYPE_F16, False, 1.0),
    "causal_b1h2n64d64_f16": (11, 1, 2, 2, 64, 64, 64, oracle.DTYPE_F16, True, 1.0),
    "gqa_b1h4kv2_m32n48d128_f16": (12, 1, 4, 2, 32, 48, 128, oracle.DTYPE_F16, False, 1.0),
    "causal_m40n70d64_bf16": (13, 2, 2, 1, 40, 70, 64, oracle.DTYPE_BF16, True, 1.0),
    "d256_b1h1m16n40_bf16": (14, 1, 1, 1, 16, 40, 256, oracle.DTYPE_BF16, False, 0.5),
    "single_key_d64_f16": (15, 1, 2, 2, 8, 1, 64, oracle.DTYPE_F16, False, 1.0),
}

GEMM_CASES = {
    "gemm_m64n96k128_f16": (21, 64, 96, 128),
    "gemm_m128n64k256_f16": (22, 128, 64, 256),
}


def attention_inputs(seed, B, H, Hkv, M, N, D, dtype, scale):
    q = oracle.round_to(oracle.portable_normal(seed, (B, H, M, D)) * scale, dtype)
    k = oracle.round_to(oracle.portable_normal(seed + 1, (B, Hkv, N, D)) * scale, dtype)
    v = oracle.round_to(oracle.portable_normal(seed + 2, (B, Hkv, N, D)) * scale, dtype)
    return q, k, v


def gemm_inputs(seed, M, N, K):
    a = oracle.round_to(oracle.portable_uniform(seed, (M, K), -1.0, 1.0), oracle.DTYPE_F16)
    b = oracle.round_to(oracle.portable_uniform(seed + 1, (K, N), -1.0, 1.0), oracle.DTYPE_F16)
    return a, b


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    return h.hexdigest()


def torch_sdpa_f64(q, k, v, causal: bool):
    qt, kt, vt = (torch.from_numpy(x).double() for x in (q, k, v))
    gqa = qt.shape[1] != kt.shape[1]
    o = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, enable_gqa=gqa)
    D = qt.shape[-1]
    kk = kt.repeat_interleave(qt.shape[1] // kt.shape[1], dim=1)
    s = (qt @ kk.transpose(-1, -2)) * D ** -0.5
    if causal:
        M, N = s.shape[-2:]
        s = s.masked_fill(torch.ones(M, N, dtype=torch.bool).tril().logical_not(), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return o.numpy(), lse.numpy()


def main() -> None:
    meta = {"attention": {}, "gemm": {}}
    for name, (seed, B, H, Hkv, M, N, D, dtype, causal, scale) in ATTENTION_CASES.items():
        q, k, v = attention_inputs(seed, B, H, Hkv, M, N, D, dtype, scale)
        o, lse = torch_sdpa_f64(q, k, v, causal)
        np.savez(HERE / f"{name}.npz", o=o.astype(np.float32), lse=lse.astype(np.float32))
        meta["attention"][name] = {
            "seed": seed, "B": B, "H": H, "Hkv": Hkv, "M": M, "N": N, "D": D, "dtype": dtype, "causal": causal,
            "input_scale": scale, "inputs_sha256": digest(q, k, v),
        }
    for name, (seed, M, N, K) in GEMM_CASES.items():
        a, b = gemm_inputs(seed, M, N, K)
        c = (torch.from_numpy(a).double() @ torch.from_numpy(b).double()).numpy()
        np.savez(HERE / f"{name}.npz", c=c.astype(np.float32))
        meta["gemm"][name] = {"seed": seed, "M": M, "N": N, "K": K, "inputs_sha256": digest(a, b)}
    meta["generator"] = f"torch {torch.__version__} CPU float64 scaled_dot_product_attention / matmul"
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(ATTENTION_CASES) + len(GEMM_CASES)} fixtures to {HERE}")


if __name__ == "__main__":
    main()
