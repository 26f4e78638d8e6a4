"""Host-side tables of the product (sub0_amd.cda.algorithm.compression)
against the reference's own values (golden fixture)."""
import numpy as np

from sub0_amd.cda.algorithm import compression as C


def test_lloyd_beta_codebooks_bit_exact(codebooks):
    assert np.array_equal(C.lloyd_max_centroids_beta(16, 128).numpy(), codebooks["lloyd_beta16"])
    assert np.array_equal(C.lloyd_max_centroids_beta(4, 128).numpy(), codebooks["lloyd_beta4"])


def test_hadamard_and_uniform_bit_exact(codebooks):
    assert np.array_equal(C.hadamard_matrix(128).numpy(), codebooks["hadamard128"])
    assert np.array_equal(C.half_rotate_pair(128).numpy(), codebooks["hadamard128"])
    for L in (16, 4):
        assert np.array_equal(C.uniform_centroids(L).numpy(), codebooks[f"uniform{L}"])


def test_compressor_tables(codebooks):
    cmp = C.Compressor(128, num_levels=16)
    assert np.array_equal(cmp.codebook.numpy(), codebooks["lloyd_beta16"])
    assert np.array_equal(cmp.rotation.numpy(), codebooks["hadamard128"])
    assert cmp.bytes_per_row == 64 and cmp.bits == 4
    assert abs(cmp.compression_ratio() - 256 / 68) < 1e-12
    c2 = C.Compressor(128, num_levels=4)
    assert c2.bytes_per_row == 32 and np.array_equal(c2.codebook.numpy(), codebooks["lloyd_beta4"])


def test_pack_helpers_match_checker():
    import torch
    from oracle import cda_oracle as O
    rng = np.random.default_rng(3)
    i4 = rng.integers(0, 16, (7, 128)).astype(np.uint8)
    i2 = rng.integers(0, 4, (7, 128)).astype(np.uint8)
    assert np.array_equal(C.pack_4bit(torch.from_numpy(i4)).numpy(), O.pack_4bit(i4))
    assert np.array_equal(C.pack_2bit(torch.from_numpy(i2)).numpy(), O.pack_2bit(i2))
    assert np.array_equal(C.unpack_4bit(torch.from_numpy(O.pack_4bit(i4)), d=128).numpy(), i4)
    assert np.array_equal(C.unpack_2bit(torch.from_numpy(O.pack_2bit(i2)), d=128).numpy(), i2)
