"""Row f1: the on-disk index (trident_amd.persist).

CPU: a saved and reloaded index holds every tensor of the built one bit for bit (with the base
from xb_sorted.bin, and from the original-order base when saved without it); interrupted or
damaged directories are refused.  GPU: a reloaded index (base in HBM and in mapped host memory)
searches exactly like the float64 oracle and like the index it was saved from."""
import os

import numpy as np
import pytest
import torch

from tests.helpers import assert_exact, build_index, oracle_search
from trident_amd import clustering, datagen, persist
from trident_amd.index import SharedClusterStorage, TridentV4Index

_TENSORS = ("centroids", "W_combined", "b_combined", "W_coarse_only", "b_coarse_only", "vmin_pad",
            "delta_pad", "eps_pad", "blk_bounds4", "tile_r_minmax", "cluster_tile_off", "sq8_packed",
            "sq8_cells", "tile_orig_ids", "vec_Ar", "vec_cn", "r_vec_sorted")
_STORAGE = ("xb_sorted", "orig_ids_sorted", "cluster_vec_off", "list_ids_sorted")


@pytest.fixture(scope="module")
def cpu_index():
    xb, _ = datagen.cfg1(N=5000, D=72, B=8, n_centers=16, seed=7)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 20, seed=0, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, 20, device="cpu")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device="cpu", max_batch=8, max_nprobe=8)
    return ix, xb.numpy(), mean64, R64


def _same_index(a, b):
    for n in ("N", "D", "D_pad", "nlist", "tile_size", "per_cluster_sq8", "total_tiles", "rot_sq_min",
              "rot_sq_max", "seed_rows"):
        assert getattr(a, n) == getattr(b, n), n
    assert a.storage.within == b.storage.within
    for n in _TENSORS:
        ta, tb = getattr(a, n), getattr(b, n)
        assert ta.dtype == tb.dtype and torch.equal(ta.cpu(), tb.cpu()), n
    for n in _STORAGE:
        assert torch.equal(getattr(a.storage, n).cpu(), getattr(b.storage, n).cpu()), n
    for x, y in zip(a.cent_band, b.cent_band):
        assert (torch.equal(x, y) if isinstance(x, torch.Tensor) else x == y)
    for n in ("fine_codes", "fine_qp"):
        ta, tb = getattr(a, n, None), getattr(b, n, None)
        assert (ta is None) == (tb is None), n
        if ta is not None:
            assert ta.dtype == tb.dtype and torch.equal(ta.cpu(), tb.cpu()), n


def test_round_trip_with_base(cpu_index, tmp_path):
    ix, _, mean64, R64 = cpu_index
    persist.save_index(ix, str(tmp_path), mean64=mean64, R64=R64)
    assert sorted(os.listdir(tmp_path)) == sorted(
        ["meta.npz", "sort_perm.bin", "sq8_packed.bin", "tile_orig_ids.bin", "vec_Ar.bin", "r_vec_sorted.bin",
         "xb_sorted.bin"])
    got = persist.load_index(str(tmp_path), device="cpu", max_batch=8, max_nprobe=8)
    _same_index(ix, got)
    with np.load(tmp_path / "meta.npz", allow_pickle=False) as z:
        assert np.array_equal(z["mean64"], mean64) and np.array_equal(z["R64"], R64)


def test_round_trip_keeps_the_row_order(tmp_path):
    """A layout ordered by residual norm within clusters is reloaded as such (the seeding pass
    then scans TridentIndexView.seed_rows rows per seeding slice)."""
    xb, _ = datagen.cfg2(N=4000, D=64, B=8, n_centers=16, seed=9)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 12, seed=0, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, 12, device="cpu", within="residual")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device="cpu", max_batch=8, max_nprobe=8)
    assert ix.seed_rows > 0
    persist.save_index(ix, str(tmp_path))
    got = persist.load_index(str(tmp_path), device="cpu", max_batch=8, max_nprobe=8)
    assert got.storage.within == "residual"
    _same_index(ix, got)


def test_round_trip_without_base(cpu_index, tmp_path):
    ix, xb, _, _ = cpu_index
    persist.save_index(ix, str(tmp_path), include_base=False)
    assert not (tmp_path / "xb_sorted.bin").exists()
    with pytest.raises(ValueError, match="xb_raw"):
        persist.load_index(str(tmp_path), device="cpu")
    got = persist.load_index(str(tmp_path), device="cpu", xb_raw=xb, max_batch=8, max_nprobe=8)
    _same_index(ix, got)


def test_round_trip_with_fine_level(tmp_path):
    xb, _ = datagen.cfg2(N=4000, D=64, B=8, n_centers=16, seed=8)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 16, seed=0, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, 16, device="cpu")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device="cpu", max_batch=8, max_nprobe=8,
                        fine_level=True)
    persist.save_index(ix, str(tmp_path))
    assert (tmp_path / "fine_codes.bin").exists() and (tmp_path / "fine_qp.bin").exists()
    _same_index(ix, persist.load_index(str(tmp_path), device="cpu", max_batch=8, max_nprobe=8))


def test_damaged_directories_are_refused(cpu_index, tmp_path):
    ix, _, _, _ = cpu_index
    with pytest.raises(ValueError, match="meta.npz"):
        persist.load_index(str(tmp_path), device="cpu")
    persist.save_index(ix, str(tmp_path))
    f = tmp_path / "vec_Ar.bin"
    with open(f, "r+b") as h:
        h.truncate(os.path.getsize(f) - 8)
    with pytest.raises(ValueError, match="vec_Ar.bin"):
        persist.load_index(str(tmp_path), device="cpu")


def test_interrupted_resave_is_refused(cpu_index, tmp_path, monkeypatch):
    """A re-save over an existing index removes its meta.npz first: interrupted before the new
    meta lands (here: the meta write fails), the directory holds no loadable index, although
    every .bin has the right size."""
    ix, _, _, _ = cpu_index
    persist.save_index(ix, str(tmp_path))

    def boom(*a, **k):
        raise OSError("interrupted")

    monkeypatch.setattr(persist.np, "savez", boom)
    with pytest.raises(OSError, match="interrupted"):
        persist.save_index(ix, str(tmp_path))
    monkeypatch.undo()
    with pytest.raises(ValueError, match="meta.npz"):
        persist.load_index(str(tmp_path), device="cpu")


def test_bin_from_another_save_is_refused(cpu_index, tmp_path):
    """Each .bin carries its save's token: a file of the right size from another save of the
    same shapes is refused."""
    ix, _, _, _ = cpu_index
    a, b = tmp_path / "a", tmp_path / "b"
    persist.save_index(ix, str(a))
    persist.save_index(ix, str(b))
    os.replace(a / "sq8_packed.bin", b / "sq8_packed.bin")
    with pytest.raises(ValueError, match="another save"):
        persist.load_index(str(b), device="cpu")


def test_inconsistent_meta_is_refused(cpu_index, tmp_path):
    """Manifest shapes and list offsets are checked against the index sizes before any copy."""
    ix, _, _, _ = cpu_index
    persist.save_index(ix, str(tmp_path))
    meta_f = tmp_path / "meta.npz"
    with np.load(meta_f, allow_pickle=False) as z:
        meta = {k: z[k] for k in z.files}

    def rewrite(**changes):
        m = dict(meta, **changes)
        np.savez(str(tmp_path / "meta.npz"), **m)

    off = meta["vec_off"].copy()
    off[-1] += 1
    rewrite(vec_off=off)
    with pytest.raises(ValueError, match="vec_off"):
        persist.load_index(str(tmp_path), device="cpu")
    shapes = meta["bin_shapes"].copy()
    i = list(map(str, meta["bin_names"])).index("vec_Ar")
    shapes[i] = f"{int(meta['N']) - 1},2"
    rewrite(bin_shapes=shapes)
    with pytest.raises(ValueError, match="vec_Ar"):
        persist.load_index(str(tmp_path), device="cpu")
    rewrite(total_tiles=np.int64(int(meta["total_tiles"]) + 1))
    with pytest.raises(ValueError, match="tile_off"):
        persist.load_index(str(tmp_path), device="cpu")
    rewrite()
    persist.load_index(str(tmp_path), device="cpu", max_batch=8, max_nprobe=8)


def test_save_after_releasing_the_packing(tmp_path):
    """An index that keeps only the batched route's cells on its device saves the reference
    packing rebuilt from them: the reload holds the same sq8_packed as the index before the
    release."""
    xb, _ = datagen.cfg2(N=3000, D=64, B=8, n_centers=16, seed=9)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 12, seed=0, niter=3)
    st = SharedClusterStorage(xb.numpy(), lid, r, 12, device="cpu")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device="cpu", max_batch=8, max_nprobe=8)
    before = ix.sq8_packed.clone()
    ix.release_packed_codes()
    assert not ix.has_packed_codes and "sq8_packed" not in ix.hbm_footprint()
    persist.save_index(ix, str(tmp_path))
    got = persist.load_index(str(tmp_path), device="cpu", max_batch=8, max_nprobe=8)
    assert torch.equal(got.sq8_packed, before) and torch.equal(got.sq8_cells, ix.sq8_cells)


def test_user_meta_round_trip(cpu_index, tmp_path):
    ix, _, _, _ = cpu_index
    persist.save_index(ix, str(tmp_path), include_base=False, user={"cfg": 4, "seed": 11, "tag": "x"})
    assert persist.read_user_meta(str(tmp_path)) == {"cfg": 4, "seed": 11, "tag": "x"}
    assert persist.read_user_meta(str(tmp_path / "nothing")) == {}


@pytest.mark.gpu
@pytest.mark.parametrize("placement", ["device", "host"])
def test_reloaded_index_searches_exactly(dev, tmp_path, placement):
    xb, xq = datagen.cfg2(N=30_000, D=128, B=256, n_centers=64, seed=71)
    b = build_index(xb, 64, dev, max_batch=256)
    persist.save_index(b.ix, str(tmp_path))
    ix2 = persist.load_index(str(tmp_path), device=dev, xb_placement=placement, max_batch=256, max_nprobe=128)
    _same_index(b.ix, ix2)
    q = torch.as_tensor(xq.numpy()).to(dev).contiguous()
    for mode, route in ((2, 1), (2, 2), (10, 0), (11, 0)):
        _, rd, ri = oracle_search(b, xq.numpy(), 16, 10)
        d1, i1, _ = b.ix.search(q, 16, mode=mode, k=10, route=route, ub_seed=1)
        d1, i1 = d1.cpu().numpy().copy(), i1.cpu().numpy().copy()
        d2, i2, _ = ix2.search(q, 16, mode=mode, k=10, route=route, ub_seed=1)
        torch.cuda.synchronize()
        assert_exact(d2.cpu().numpy(), i2.cpu().numpy(), rd, ri, f"reloaded mode {mode} route {route}")
        assert np.array_equal(d1, d2.cpu().numpy()) and np.array_equal(i1, i2.cpu().numpy())
    if ix2.storage._host_buf is not None:
        torch.cuda.synchronize()
        ix2.storage._host_buf.free()
