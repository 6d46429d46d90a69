"""Row f2: the pipelined search (trident_amd.pipeline) returns, for every query of a host
query set, exactly what a single-batch search returns -- the float64 oracle's ids and rounded
distances -- with several batches in flight on separate streams, a ragged last batch, both
mode-2 routes and the base in HBM or in mapped host memory."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_exact, build_index, oracle_search
from trident_amd import datagen
from trident_amd.pipeline import SearchPipeline

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["device", "host"])
def pipe_set(dev, request):
    xb, xq = datagen.cfg2(N=40_000, D=128, B=2_300, n_centers=64, seed=81)
    b = build_index(xb, 96, dev, max_batch=1024, xb_placement=request.param)
    yield b, xq.numpy()
    if b.ix.storage._host_buf is not None:
        torch.cuda.synchronize()
        b.ix.storage._host_buf.free()


@pytest.mark.parametrize("route,depth,batch", [(1, 2, 512), (2, 3, 700), (0, 1, 1024), (2, 4, 97)])
def test_pipeline_matches_oracle(pipe_set, route, depth, batch):
    b, xq = pipe_set
    nprobe, K = 12, 10
    _, rd, ri = oracle_search(b, xq, nprobe, K)
    pipe = SearchPipeline(b.ix, nprobe, K, batch=batch, depth=depth, route=route, ub_seed=1)
    d, i = pipe.run(xq)
    assert_exact(d, i, rd, ri, f"pipeline route={route} depth={depth} batch={batch}")
    d2, i2 = pipe.run(xq[:5])  # a second run, one partial batch
    assert np.array_equal(d2, d[:5]) and np.array_equal(i2, i[:5])


def test_pipeline_other_modes(pipe_set):
    b, xq = pipe_set
    for mode in (10, 11):
        _, rd, ri = oracle_search(b, xq[:900], 6, 16)
        d, i = SearchPipeline(b.ix, 6, 16, batch=256, depth=3, mode=mode).run(xq[:900])
        assert_exact(d, i, rd, ri, f"pipeline mode {mode}")


def test_pipeline_straight_after_index_build(dev):
    """The slot streams wait for the caller's stream: a pipeline started right after the index
    constructor (whose last kernels -- the cluster bound table among them -- are still queued on
    the current stream, with no synchronisation in between) sees the finished index."""
    from trident_amd import clustering
    from trident_amd.index import SharedClusterStorage, TridentV4Index

    xb, xq = datagen.cfg2(N=30_000, D=128, B=1_500, n_centers=48, seed=93)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 64, seed=0, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, 64, device=dev)
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device=dev, max_batch=512,
                        max_nprobe=16, k=10)
    with SearchPipeline(ix, 8, 10, batch=512, depth=3, route=2, ub_seed=1) as pipe:
        d, i = pipe.run(xq.numpy())
    h = ix.host_arrays()
    cids, _ = O.coarse_probe(np.ascontiguousarray(xq.numpy()), h["centroids"], 8)
    rd, ri = O.ivf_exact(np.ascontiguousarray(xq.numpy()), cids, h["vec_off"], h["xb_sorted"],
                         h["orig_ids_sorted"], 10)
    assert_exact(d, i, rd, ri, "pipeline straight after the build")
