"""Write the golden fixtures under tests/golden/ from the reference oracle.

Run once, in the build container, where the reference is mounted read-only:

    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-torch algorithm modules
(``cda/algorithm/compression.py`` and ``cda/algorithm/attention.py``) on the
CPU and records their inputs and outputs as small ``.npz`` files.  Only data
is written: no reference source travels with the repository.  The functions
whose exact values only the reference itself can pin are:

* ``lloyd_max_centroids_beta`` (torch CPU RNG stream, ``compression.py:86-113``);
* ``Compressor.encode`` last-ulp behaviour (MKL sgemm order, ``Tensor.norm``
  reduction order, ``compression.py:287-335``);
* ``attention_compressed`` and the split-K contract
  (``attention.py:190-272, 306-346, 387-482``), pinned to a tolerance.

The tests under ``tests/`` read the fixtures; they never import the reference.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))

from oracle import synth  # noqa: E402


def _sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from cda.algorithm import attention as A
    from cda.algorithm import compression as C

    torch.set_num_threads(8)
    D = 128

    # ---- codebooks -------------------------------------------------------
    cb16 = C.lloyd_max_centroids_beta(16, D)
    cb4 = C.lloyd_max_centroids_beta(4, D)
    np.savez(HERE / "codebooks.npz",
             lloyd_beta16=cb16.numpy(), lloyd_beta4=cb4.numpy(),
             uniform16=C.uniform_centroids(16).numpy(),
             uniform4=C.uniform_centroids(4).numpy(),
             hadamard128=C.hadamard_matrix(D).numpy())

    # ---- quantize_unit: ties, exact centroids, range ends ----------------
    qrows = {}
    for name, cb in (("cb16", cb16), ("cb4", cb4)):
        mids = ((cb[:-1] + cb[1:]) * 0.5)
        xs = torch.cat([
            cb, mids, torch.nextafter(mids, torch.full_like(mids, 2.0)),
            torch.nextafter(mids, torch.full_like(mids, -2.0)),
            torch.tensor([-1.0, 1.0, 0.0, -0.0]),
            torch.linspace(-1.0, 1.0, 4001),
        ]).float()
        cmp = C.Compressor(D, num_levels=cb.numel(), codebook=cb)
        qrows[f"{name}_x"] = xs.numpy()
        qrows[f"{name}_idx"] = cmp.quantize_unit(xs).numpy()
    np.savez(HERE / "quantize.npz", **qrows)

    # ---- encode: K4 and K2 on outlier data plus edge rows -----------------
    x = synth.kv_with_outliers(1001, (1024, D))
    edge = np.zeros((8, D), dtype=np.float16)
    edge[1, :] = 1.0                                      # constant row
    edge[2, :] = np.float16(6.0e-8)                       # subnormal row
    edge[3, ::2] = 60000.0                                # huge values
    edge[3, 1::2] = -60000.0
    edge[4, 7] = 1.0                                      # one-hot (rotation spreads it)
    edge[5, :] = np.arange(D, dtype=np.float16) / 64.0
    edge[6, :64] = 0.5
    edge[6, 64:] = -0.5
    # row 0 stays all-zero: norm clamps to 1e-12
    xall = np.concatenate([x, edge]).astype(np.float16)
    xt = torch.from_numpy(xall)
    enc = {"x": xall}
    for levels, tag in ((16, "k4"), (4, "k2")):
        cb = cb16 if levels == 16 else cb4
        cmp = C.Compressor(D, num_levels=levels, codebook=cb)
        slot = cmp.encode(xt)
        enc[f"{tag}_idx"] = slot.idx.numpy()
        enc[f"{tag}_norm"] = slot.norm.numpy()
        enc[f"{tag}_dec_rot"] = cmp.decode(slot, rotated=True).numpy()
    cmp16 = C.Compressor(D, num_levels=16, codebook=cb16)
    enc["x_rot"] = cmp16.rotate(xt).numpy()
    cmpu = C.Compressor(D, num_levels=16, codebook_mode="uniform")
    su = cmpu.encode(xt[:256])
    enc["uniform_k4_idx"] = su.idx.numpy()
    enc["uniform_k4_norm"] = su.norm.numpy()
    np.savez_compressed(HERE / "encode.npz", **enc)

    # ---- attention: small GQA shapes -------------------------------------
    def attn_case(seed, B, H_q, H_kv, N, M_q=1, causal=False, k_splits=3):
        g = H_q // H_kv
        k = torch.from_numpy(synth.kv_with_outliers(seed, (B, H_kv, N, D)))
        v = torch.from_numpy(synth.normal_f16(seed + 1, (B, H_kv, N, D)))
        q = torch.from_numpy(synth.normal_f16(seed + 2, (B, H_q, M_q, D)))
        cK = C.Compressor(D, num_levels=16, codebook=cb16)
        cV = C.Compressor(D, num_levels=16, codebook=cb16)
        ks, vs = cK.encode(k), cV.encode(v)
        q_off = N - M_q if causal else 0
        out = A.attention_compressed(q, ks, vs, cmp_K=cK, cmp_V=cV, group_size=g,
                                     causal=causal, q_offset=q_off)
        q_rot = cK.rotate(q)
        out_rot = A.attention_compressed(q_rot, ks, vs, cmp_K=cK, cmp_V=cV,
                                         group_size=g, causal=causal,
                                         q_offset=q_off, rotated=True)
        split = A.attention_compressed_split_reference(
            q_rot, ks, vs, cmp_K=cK, cmp_V=cV, group_size=g, k_splits=k_splits,
            causal=causal, q_offset=q_off)
        o_un, m, l = A.attention_compressed_partial_reference(
            q_rot, ks, vs, cmp_K=cK, cmp_V=cV, group_size=g, causal=causal,
            q_offset=q_off, key_start=N // 3, key_end=N - N // 5)
        return dict(q=q.numpy(),
                    k_idx=ks.idx.numpy(), k_norm=ks.norm.numpy(),
                    v_idx=vs.idx.numpy(), v_norm=vs.norm.numpy(),
                    q_rot=q_rot.numpy(), out=out.numpy(), out_rot=out_rot.numpy(),
                    split_out=split.numpy(), part_o=o_un.numpy(), part_m=m.numpy(),
                    part_l=l.numpy(),
                    meta=np.array([B, H_q, H_kv, N, M_q, int(causal), q_off,
                                   k_splits, N // 3, N - N // 5]))

    np.savez_compressed(HERE / "attn_gs4.npz", **attn_case(2001, 2, 8, 2, 300))
    np.savez_compressed(HERE / "attn_gs8.npz", **attn_case(2002, 1, 16, 2, 77, k_splits=4))
    np.savez_compressed(HERE / "attn_causal.npz",
                        **attn_case(2003, 1, 8, 2, 200, M_q=37, causal=True))

    # ---- config 0 (B=1, 32/8 heads, N=4096): encodings + output -----------
    B, H_q, H_kv, N = 1, 32, 8, 4096
    seed = synth.cfg_seed(B, N)
    k = torch.from_numpy(synth.kv_with_outliers(seed, (B, H_kv, N, D)))
    v = torch.from_numpy(synth.normal_f16(seed + 1, (B, H_kv, N, D)))
    q = torch.from_numpy(synth.normal_f16(seed + 2, (B, H_q, 1, D)))
    cK = C.Compressor(D, num_levels=16, codebook=cb16)
    cV = C.Compressor(D, num_levels=16, codebook=cb16)
    ks, vs = cK.encode(k), cV.encode(v)
    out = A.attention_compressed(q, ks, vs, cmp_K=cK, cmp_V=cV, group_size=H_q // H_kv)
    np.savez_compressed(HERE / "attn_cfg0.npz", out=out.numpy(), q=q.numpy(),
                        k_idx=ks.idx.numpy(), k_norm=ks.norm.numpy(),
                        v_idx=vs.idx.numpy(), v_norm=vs.norm.numpy())
    meta = dict(B=B, H_q=H_q, H_kv=H_kv, N=N, seed=seed,
                k_sha=_sha(ks.idx.numpy(), ks.norm.numpy()),
                v_sha=_sha(vs.idx.numpy(), vs.norm.numpy()),
                torch=torch.__version__,
                note="inputs regenerate from oracle/synth.py with the seeds "
                     "seed (K, outliers), seed+1 (V), seed+2 (q)")
    (HERE / "attn_cfg0.json").write_text(json.dumps(meta, indent=1) + "\n")
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
