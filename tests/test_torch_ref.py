"""The torch-CPU restatement (oracle/torch_ref.py, the CPU baseline bench.py
times) against the reference-written fixtures: it must give the reference's
bits on this host's CPU."""
import json
from pathlib import Path

import numpy as np
import torch

from oracle import synth
from oracle import torch_ref as T

GOLD = Path(__file__).parent / "golden"


def test_hadamard_equals_reference(codebooks):
    assert np.array_equal(T.hadamard().numpy(), codebooks["hadamard128"])


def test_encode_rows_equal_reference(golden, codebooks):
    e = golden("encode.npz")
    cb = torch.from_numpy(codebooks["lloyd_beta16"])
    codes, norm = T.encode(torch.from_numpy(e["x"]), cb, T.hadamard())
    assert np.array_equal(codes.numpy(), e["k4_idx"])
    assert np.array_equal(norm.numpy().view(np.uint32), e["k4_norm"].view(np.uint32))
    dec = T.decode_rows(torch.from_numpy(e["k4_idx"]), torch.from_numpy(e["k4_norm"]), cb)
    assert np.array_equal(dec.numpy().view(np.uint16), e["k4_dec_rot"].view(np.uint16))


def test_config0_equals_reference(golden, codebooks):
    g = golden("attn_cfg0.npz")
    meta = json.loads((GOLD / "attn_cfg0.json").read_text())
    seed, N = meta["seed"], meta["N"]
    cb = torch.from_numpy(codebooks["lloyd_beta16"])
    H = T.hadamard()
    k = torch.from_numpy(synth.kv_with_outliers(seed, (1, 8, N, 128)))
    v = torch.from_numpy(synth.normal_f16(seed + 1, (1, 8, N, 128)))
    kc, kn = T.encode(k, cb, H)
    vc, vn = T.encode(v, cb, H)
    assert np.array_equal(kc.numpy(), g["k_idx"]) and np.array_equal(vc.numpy(), g["v_idx"])
    assert np.array_equal(kn.numpy(), g["k_norm"]) and np.array_equal(vn.numpy(), g["v_norm"])
    out = T.attention_compressed(torch.from_numpy(g["q"]), kc, kn, vc, vn, cb, H, 4)
    assert np.array_equal(out.numpy().view(np.uint16), g["out"].view(np.uint16))
