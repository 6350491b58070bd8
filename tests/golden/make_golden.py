"""Write the golden fixtures in this directory from the reference implementation.

Run ONCE in the build container, where the reference is mounted read-only:

    python tests/golden/make_golden.py /root/reference/src

It imports the reference's own functions (nothing from this repository) and
records their inputs and outputs as data:

* ``params.json``      -- fp32 codebooks (D=128, bits 1..4) and SHA-256 of the
                          rotation matrices (seeds 0, 1) and the QJL matrix
                          (seed 31337), plus a few of their entries.
* ``encode_small.npz`` -- bf16 inputs and the packed outputs of the
                          reference's ``_encode_group`` / ``_encode_keys_qjl_group``
                          (CPU torch path) for Q_mse 2/3/4-bit and Q_prod 4-bit.
* ``attention_small.npz`` -- a packed layer built by the reference's
                          ``initialize_from_dense`` and the output of its
                          ``chunked_turboquant_attention`` (CPU path) for
                          Q_prod 4-bit and Q_mse 3-bit.

The fixtures are consumed by ``tests/test_oracle_golden.py``; nothing at
test time (and nothing on the GPU box) reads the reference.
"""

from __future__ import annotations

import hashlib
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
D = 128


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def synth_kv(gen: torch.Generator, b: int, h: int, n: int, mu: float = math.log(20.0), sigma: float = 0.3) -> torch.Tensor:
    """Direction iid N(0,1) normalised; norm lognormal(mu, sigma); cast to bf16."""
    d = torch.randn(b, h, n, D, generator=gen)
    d = d / d.norm(dim=-1, keepdim=True)
    nrm = torch.exp(mu + sigma * torch.randn(b, h, n, generator=gen))
    return (d * nrm[..., None]).to(torch.bfloat16)


def main(ref_src: str) -> None:
    sys.path.insert(0, ref_src)
    from turboquant.quantization.turboquant_mse import build_scalar_codebook, random_rotation_matrix
    from turboquant.runtime import packed_qmse_cache as pqc
    from turboquant.runtime.attention import chunked_turboquant_attention

    torch.set_num_threads(1)

    # ---------------------------------------------------------------- params
    params: dict = {"dimension": D, "codebooks": {}, "rotations": {}, "qjl": {}}
    for bits in (1, 2, 3, 4):
        cb = build_scalar_codebook(dimension=D, bits=bits, grid_size=32769)
        params["codebooks"][str(bits)] = {
            "centers_f64": [float(x) for x in cb.centers],
            "boundaries_f64": [float(x) for x in cb.boundaries],
            "centers_f32_hex": [np.float32(x).tobytes().hex() for x in cb.centers],
            "boundaries_f32_hex": [np.float32(x).tobytes().hex() for x in cb.boundaries],
        }
    for seed in (0, 1):
        r = random_rotation_matrix(dimension=D, seed=seed)
        params["rotations"][str(seed)] = {
            "sha256": hashlib.sha256(np.ascontiguousarray(r).tobytes()).hexdigest(),
            "r00": float(r[0, 0]), "r01": float(r[0, 1]), "r_last": float(r[-1, -1]),
        }
    for seed in (31337,):
        s = pqc._generate_qjl_matrix(D, seed)
        params["qjl"][str(seed)] = {
            "sha256": hashlib.sha256(s.numpy().tobytes()).hexdigest(),
            "s00": float(s[0, 0]), "s01": float(s[0, 1]), "s_last": float(s[-1, -1]),
        }
    (HERE / "params.json").write_text(json.dumps(params, indent=1))

    def tensors(bits: int, seed: int):
        cb = build_scalar_codebook(dimension=D, bits=bits, grid_size=32769)
        rot = torch.from_numpy(random_rotation_matrix(dimension=D, seed=seed)).to(torch.float32)
        return rot, torch.from_numpy(cb.centers.astype("float32")), torch.from_numpy(cb.boundaries.astype("float32"))

    # ---------------------------------------------------------------- encode
    gen = torch.Generator().manual_seed(1234)
    x = synth_kv(gen, 1, 2, 60)
    # special rows: an all-zero vector, a tiny vector, a huge-norm vector, a one-hot vector
    extra = torch.zeros(1, 2, 4, D)
    extra[0, 0, 1] = 1e-3 * torch.randn(D, generator=gen)
    extra[0, 0, 2] = 3000.0 * torch.randn(D, generator=gen) / math.sqrt(D)
    extra[0, 0, 3, 5] = 7.0
    extra[0, 1] = torch.randn(4, D, generator=gen)
    x = torch.cat((x, extra.to(torch.bfloat16)), dim=2)  # [1, 2, 64, D]
    enc: dict[str, np.ndarray] = {"x_bf16": _bf16_bits(x)}
    for bits, seed in ((2, 0), (3, 0), (4, 0)):
        rot, c, bnd = tensors(bits, seed)
        p = pqc.PackedMSELayer._encode_group(x, rot, c, bnd, bits)
        enc[f"mse{bits}_codes"] = p.packed_indices.numpy().copy()
        enc[f"mse{bits}_norms"] = _f16_bits(p.norms)
    # Q_prod at total 4 bits: keys use the 3-bit codebook with R(seed+1) and S(seed+31337)
    rot, c, bnd = tensors(3, 1)
    smat = pqc._generate_qjl_matrix(D, 31337)

    class _Enc:
        _encode_group = staticmethod(pqc.PackedMSELayer._encode_group)
        _decode_group = staticmethod(pqc.PackedMSELayer._decode_group)

    mse, qjl = pqc.PackedMSELayer._encode_keys_qjl_group(_Enc(), x, rot, c, bnd, 3, smat)
    enc["prod4_codes"] = mse.packed_indices.numpy().copy()
    enc["prod4_norms"] = _f16_bits(mse.norms)
    enc["prod4_signs"] = qjl.packed_signs.numpy().copy()
    enc["prod4_rnorms"] = _f16_bits(qjl.residual_norms)
    dec = pqc.PackedMSELayer._decode_group(mse, rot, c)
    enc["prod4_khat_bf16"] = _bf16_bits(dec)
    full = pqc.PackedMSELayer._decode_keys_qjl_group(_Enc(), mse, qjl, rot, c, smat)
    enc["prod4_kfull_bf16"] = _bf16_bits(full)
    np.savez_compressed(HERE / "encode_small.npz", **enc)

    # ------------------------------------------------------------- attention
    class _Layer(pqc.PackedMSELayer):
        def get_max_length(self) -> int:  # abstract in newer transformers
            return -1

    att: dict[str, np.ndarray] = {}
    cases = (("prod4", 4, True, 8, 2, 1100), ("mse3", 3, False, 8, 2, 700))
    for name, bits, qjl_keys, hq, hkv, n in cases:
        g = torch.Generator().manual_seed(4321 + bits)
        k = synth_kv(g, 1, hkv, n)
        v = synth_kv(g, 1, hkv, n)
        q = torch.randn(1, hq, 1, D, generator=g).to(torch.bfloat16)
        layer = _Layer(bits=bits, seed=0, use_qjl_keys=qjl_keys, quantize_decode=True)
        layer.initialize_from_dense(k, v)
        out = chunked_turboquant_attention(q, layer, n_kv_groups=hq // hkv)
        att[f"{name}_q_bf16"] = _bf16_bits(q)
        att[f"{name}_kcodes"] = layer.keys_packed.packed_indices.numpy().copy()
        att[f"{name}_knorms"] = _f16_bits(layer.keys_packed.norms)
        att[f"{name}_vcodes"] = layer.values_packed.packed_indices.numpy().copy()
        att[f"{name}_vnorms"] = _f16_bits(layer.values_packed.norms)
        if qjl_keys:
            att[f"{name}_signs"] = layer._keys_qjl.packed_signs.numpy().copy()
            att[f"{name}_rnorms"] = _f16_bits(layer._keys_qjl.residual_norms)
        att[f"{name}_out_bf16"] = _bf16_bits(out)
        att[f"{name}_meta"] = np.array([bits, int(qjl_keys), hq, hkv, n], dtype=np.int64)
    np.savez_compressed(HERE / "attention_small.npz", **att)
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
