"""Weight loaders of engine.py (CPU): the three reference layouts written from
the same synthetic tensors load back to identical [out][in] tensors.
  (A) directory tree of e2e_validate.cpp:37-84,126
  (B) CudaEngine::set_layer_weights flat vector, cuda_engine.cu:244-298
  (C) export_real_weights.py layer_XX.bin (matrices stored [in][out])
Small shapes are not possible (the loaders know the model's shapes), so each
check writes two layers (one linear, one full) of the real sizes."""
import importlib.util
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _em():
    spec = importlib.util.spec_from_file_location("qw_engine", os.path.join(ROOT, "qwen3.5_0.8b_deploy_amd", "engine.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _layer(em, i, rng):
    L = {n: rng.standard_normal(s).astype(np.float32) for n, s in em._COMMON}
    L.update({n: rng.standard_normal(s).astype(np.float32) for n, s in (em._LINEAR if em.is_linear_layer(i) else em._FULL)})
    return L


def _eq(a, b):
    assert set(a) == set(b)
    for k in a:
        assert a[k].shape == b[k].shape and np.array_equal(a[k], b[k]), k


def test_layout_b_engine_flat():
    em = _em()
    rng = np.random.default_rng(1)
    for i in (2, 3):
        L = _layer(em, i, rng)
        other = _layer(em, i + 1 if i == 2 else 2, rng)  # the section the layer type does not use
        secs = {**other, **L}
        flat = np.concatenate([secs[n].ravel() for n, _ in em._COMMON + em._LINEAR + em._FULL])
        assert flat.size == em.flat_layer_size("engine")
        _eq(em.layer_from_engine_flat(flat, i), L)


def test_layout_c_export_files(tmp_path):
    em = _em()
    rng = np.random.default_rng(2)
    layers = [_layer(em, i, rng) for i in range(4)]
    for i, L in enumerate(layers):
        fields = em._COMMON + (em._LINEAR if em.is_linear_layer(i) else em._FULL)
        # what export_real_weights.py writes: every matrix transposed to [in][out], conv1d as is
        parts = [(L[n].T if (len(s) == 2 and n != "conv") else L[n]).ravel() for n, s in fields]
        np.concatenate(parts).astype("<f4").tofile(tmp_path / f"layer_{i:02d}.bin")
        assert sum(p.size for p in parts) == em.flat_layer_size("linear" if em.is_linear_layer(i) else "full")
    fn = rng.standard_normal(em.H).astype(np.float32)
    emb = rng.standard_normal((64, em.H)).astype(np.float32)
    fn.tofile(tmp_path / "norm.bin")
    emb.tofile(tmp_path / "embedding.bin")
    got, gfn, gemb = em.load_export_files(str(tmp_path), num_layers=4)
    for a, b in zip(got, layers):
        _eq(a, b)
    assert np.array_equal(gfn, fn) and np.array_equal(gemb, emb)


def test_layout_a_dir_tree(tmp_path):
    em = _em()
    rng = np.random.default_rng(3)
    layers = [_layer(em, i, rng) for i in range(4)]
    for i, L in enumerate(layers):
        d = tmp_path / "language_backbone" / f"layer_{i}"
        d.mkdir(parents=True)
        for n, a in L.items():
            a.astype("<f4").tofile(d / (em._DIR_NAMES[n] + ".bin"))
    fn = rng.standard_normal(em.H).astype(np.float32)
    fn.tofile(tmp_path / "language_backbone" / "final_norm.bin")
    (tmp_path / "language").mkdir()
    emb = rng.standard_normal((32, em.H)).astype(np.float32)
    emb.tofile(tmp_path / "language" / "embed_tokens.bin")
    got, gfn, gemb = em.load_dir_tree(str(tmp_path), num_layers=4)
    for a, b in zip(got, layers):
        _eq(a, b)
    assert np.array_equal(gfn, fn) and np.array_equal(gemb, emb)


def test_truncated_files_are_rejected(tmp_path):
    em = _em()
    import pytest
    with pytest.raises(ValueError):
        em.layer_from_engine_flat(np.zeros(10, np.float32), 0)
    np.zeros(em.H - 1, "<f4").tofile(tmp_path / "norm.bin")
    with pytest.raises(ValueError):
        em._read_f32(str(tmp_path / "norm.bin"), em.H)
