"""On-disk formats (host side): positional reads of ``layer-NN.npz`` and
safetensors files, dimension inference and the codebook hash check, against
files written the way the reference writes them (``np.savez`` of stacked
arrays, ``scripts/runpod/v41_reap/keep_quant.py:125-133``; safetensors with a
``quantization_config`` metadata entry, ``src/keep/io/load.py:102-182``)."""

import json

import numpy as np
import pytest

from keep_amd import loaders

E, N, K, G = 5, 64, 128, 32


def _layer_arrays(rng, code_bits=16):
    out = {}
    for proj, (n, k) in (("w1", (N, K)), ("w3", (N, K)), ("w2", (K, N))):
        dt = np.uint16 if code_bits == 16 else np.uint8
        out[f"{proj}_codes"] = rng.integers(0, np.iinfo(dt).max + 1, size=(E, n, k // 8), dtype=dt)
        out[f"{proj}_scales"] = rng.random((E, n, k // G)).astype(np.float16)
    return out


def test_layer_npz_positional_reads(tmp_path):
    rng = np.random.default_rng(1)
    arrays = _layer_arrays(rng)
    path = tmp_path / "layer-00.npz"
    np.savez(path, code_bits=np.asarray(16), **arrays)
    lf = loaders.LayerFile(path)
    assert lf.code_bits == 16 and lf.num_experts == E
    assert lf.dims("w1") == (K, N, G) and lf.dims("w2") == (N, K, G)
    raw = path.read_bytes()
    for name, a in arrays.items():
        np.testing.assert_array_equal(lf.read(name), a)
        np.testing.assert_array_equal(lf.read(name, [3, 0]), a[[3, 0]])
        off, size = lf.slab(name, 4)
        assert raw[off:off + size] == a[4].tobytes()
    with pytest.raises(IndexError):
        lf.slab("w1_codes", E)
    with pytest.raises(KeyError):
        lf.read("w4_codes")


def test_layer_npz_variants_and_rejections(tmp_path):
    rng = np.random.default_rng(2)
    arrays = _layer_arrays(rng)
    p = tmp_path / "nobits.npz"
    np.savez(p, **arrays)  # the first E8P runs wrote no code_bits
    assert loaders.LayerFile(p).code_bits == 16
    a8 = _layer_arrays(rng, code_bits=8)
    p8 = tmp_path / "e8.npz"
    np.savez(p8, code_bits=np.asarray(8), **a8)
    lf8 = loaders.LayerFile(p8)
    assert lf8.code_bits == 8 and lf8.dims("w3") == (K, N, G)
    np.testing.assert_array_equal(lf8.read("w2_codes", [1]), a8["w2_codes"][[1]])
    bad = tmp_path / "mixed.npz"
    np.savez(bad, code_bits=np.asarray(8), **arrays)  # uint16 codes said to be 8-bit
    with pytest.raises(ValueError):
        loaders.LayerFile(bad).dims("w1")
    comp = tmp_path / "compressed.npz"
    np.savez_compressed(comp, code_bits=np.asarray(16), **arrays)
    with pytest.raises(ValueError, match="compressed"):
        loaders.LayerFile(comp)
    fort = tmp_path / "fortran.npz"
    np.savez(fort, w1_codes=np.asfortranarray(arrays["w1_codes"]))
    with pytest.raises(ValueError, match="Fortran"):
        loaders.LayerFile(fort)


def test_codebook_hashes_are_the_reference_tables():
    assert loaders.codebook_sha256(16) == "efc2c03c60acd955dc812ff2bade9ec6cc31259807e48473506161f3a9a230ce"
    assert loaders.codebook_sha256(8) == "b78586631069e239d29c146538722d763f4a0040d59a800e8c918ecef03e2180"
    with pytest.raises(ValueError):
        loaders.codebook_sha256(4)


def test_safetensors_dims_and_hash(tmp_path):
    from safetensors.numpy import save_file

    rng = np.random.default_rng(3)
    codes = rng.integers(0, 1 << 16, size=(E, N, K // 8), dtype=np.uint16)
    scales = rng.random((E, N, K // G)).astype(np.float16)
    meta = {"quantization_config": json.dumps({"codebook": {"sha256": loaders.codebook_sha256(16)}})}
    p = tmp_path / "m.safetensors"
    save_file({"mlp.experts.codes": codes, "mlp.experts.scales": scales,
               "lin.codes": codes[0], "lin.scales": scales[0], "bad.codes": codes.astype(np.int32),
               "bad.scales": scales}, str(p), metadata=meta)
    st = loaders.SafetensorsFile(p)
    loaders.validate_codebook_hash(st.metadata)
    assert st.infer_vq_switch_linear_dims("mlp.experts") == (K, N, E, G, 16)
    assert st.infer_vq_linear_dims("lin") == (K, N, G, 16)
    np.testing.assert_array_equal(st.read("mlp.experts.codes", [2]), codes[[2]])
    np.testing.assert_array_equal(st.read("mlp.experts.scales"), scales)
    with pytest.raises(ValueError):
        st.infer_vq_switch_linear_dims("lin")  # 2-D codes
    with pytest.raises(ValueError):
        st.infer_vq_linear_dims("mlp.experts")  # 3-D codes
    with pytest.raises(ValueError):
        st.infer_vq_switch_linear_dims("bad")  # int32 codes
    with pytest.raises(KeyError):
        st.infer_vq_switch_linear_dims("missing")
    loaders.validate_codebook_hash({})
    loaders.validate_codebook_hash({"quantization_config": json.dumps({"codebook": {"sha256": loaders.codebook_sha256(8)}})})
    with pytest.raises(ValueError, match="not supported"):
        loaders.validate_codebook_hash({"quantization_config": json.dumps({"codebook": {"sha256": "0" * 64}})})
