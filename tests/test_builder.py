"""Index layout producer (CPU torch): closed forms and invariants of the SQ8 layout.

Reference layout: benchmarks/phase4a_suite.py:95-278.  Pinned here:
  * W_combined / b_combined structure ([-2 C^T | R | 0], [|c|^2 | b | 0]) and exact centroid
    recovery c = -0.5 W;
  * rotation bounds bracket the squared singular values of the float32 rotation;
  * codes equal the closed form clip(round_half_even((x32 - vmin) / delta), 0, 255);
  * eps bounds the quantisation error of every vector against the float64 rotation;
  * unpacking sq8_packed / tile_orig_ids recovers every code and id (the wave64 layout), and
    the batched route's 16-byte cells (sq8_cells) decode to the same codes;
  * block bounds (uniform and variable schemes);
  * the Stage Y / Stage X bound arithmetic, restated in float32 numpy, brackets the float64
    distance: lb <= d64 <= ub.
"""
import math

import numpy as np
import pytest
import torch

from trident_amd import clustering, datagen
from trident_amd.index import SharedClusterStorage, TridentV4Index, choose_tile


def build(xb, nlist, T=64, var_block=0, per_cluster=1, seed=0):
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, nlist, seed=seed, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, nlist, device="cpu")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=T, per_cluster_sq8=per_cluster, var_block=var_block,
                        device="cpu", max_batch=8, max_nprobe=8)
    return ix, cen, lid


@pytest.fixture(scope="module")
def hist_ix():
    xb, xq = datagen.cfg2(N=6000, D=128, B=16, n_centers=32, seed=3)
    ix, cen, lid = build(xb, 24)
    return ix, xb.numpy(), xq.numpy(), cen, lid


@pytest.fixture(scope="module")
def gmm_ix():
    xb, xq = datagen.cfg1(N=5000, D=72, B=16, n_centers=16, seed=4)
    ix, cen, lid = build(xb, 20)
    return ix, xb.numpy(), xq.numpy(), cen, lid


def test_choose_tile():
    assert choose_tile(128) == 64 and choose_tile(96) == 64 and choose_tile(256) == 256 and choose_tile(960) == 256


def test_fused_projection_layout(gmm_ix):
    ix, _, _, cen, _ = gmm_ix
    nlist, D, D_pad = ix.nlist, ix.D, ix.D_pad
    W, b = ix.W_combined.numpy(), ix.b_combined.numpy()[0]
    assert W.shape == (D, nlist + D_pad) and D_pad == 96
    assert np.array_equal(-0.5 * W[:, :nlist].T, cen)          # exact centroid recovery
    assert np.allclose(b[:nlist], (cen.astype(np.float64) ** 2).sum(1), rtol=1e-6)
    assert np.all(W[:, nlist + D:] == 0) and np.all(b[nlist + D:] == 0)
    R = W[:, nlist:nlist + D].astype(np.float64)
    s = np.linalg.svd(R, compute_uv=False)
    assert ix.rot_sq_min <= s.min() ** 2 <= s.max() ** 2 <= ix.rot_sq_max
    assert abs(ix.rot_sq_max - 1) < 1e-5 and abs(1 - ix.rot_sq_min) < 1e-5
    assert np.abs(R.T @ R - np.eye(D)).max() < 1e-5


def rotated64(ix):
    """Base rotated in float64 with the stored float32 map, in sorted order."""
    W = ix.W_combined.numpy().astype(np.float64)
    R = W[:, ix.nlist:ix.nlist + ix.D]
    b = ix.b_combined.numpy()[0, ix.nlist:ix.nlist + ix.D].astype(np.float64)
    xs = ix.storage.xb_sorted.numpy().astype(np.float64)
    out = np.zeros((ix.N, ix.D_pad))
    out[:, :ix.D] = xs @ R + b
    return out


def unpack_codes(ix):
    """[N, D_pad] uint8 codes recovered from sq8_packed [tiles, D4, T] in sorted order."""
    T, D4 = ix.tile_size, ix.D4
    sq = ix.sq8_packed.numpy().view(np.uint32)            # [tiles, D4, T]
    toff = ix.cluster_tile_off.numpy()
    voff = ix.storage.cluster_vec_off.numpy()
    codes = np.zeros((ix.N, ix.D_pad), np.uint8)
    oids = np.zeros(ix.N, np.int64)
    for c in range(ix.nlist):
        for v in range(voff[c], voff[c + 1]):
            li = v - voff[c]
            t, s = toff[c] + li // T, li % T
            words = sq[t, :, s]                           # word d4 packs dims 4*d4 .. 4*d4+3
            codes[v] = np.stack([(words >> (8 * j)) & 0xFF for j in range(4)], 1).reshape(-1).astype(np.uint8)
            oids[v] = ix.tile_orig_ids.numpy()[t, s]
    return codes, oids


def test_codes_closed_form_and_packing(hist_ix):
    ix, xb, _, _, lid = hist_ix
    xr64 = rotated64(ix)
    xr32 = xr64.astype(np.float32)
    lid_s = ix.storage.list_ids_sorted.numpy().astype(np.int64)
    vmin, delta = ix.vmin_pad.numpy(), ix.delta_pad.numpy()
    expect = np.clip(np.round((xr32 - vmin[lid_s]) / delta[lid_s]), 0, 255).astype(np.uint8)
    codes, oids = unpack_codes(ix)
    assert np.array_equal(codes, expect)
    assert np.array_equal(oids, ix.storage.orig_ids_sorted.numpy())
    # padded tile slots are -1
    T = ix.tile_size
    assert (ix.tile_orig_ids.numpy() >= 0).sum() == ix.N
    assert ix.sq8_packed.shape == (ix.total_tiles, ix.D4, T)
    # vmin/delta closed form per cluster
    for c in range(ix.nlist):
        m = lid_s == c
        if m.any():
            assert np.array_equal(vmin[c], xr32[m].min(0))
            assert np.array_equal(delta[c], np.maximum((xr32[m].max(0) - xr32[m].min(0)) / np.float32(255.0),
                                                       np.float32(1e-12)))


def unpack_cells(ix):
    """[N, D_pad] uint8 codes recovered from sq8_cells [tiles, T/V, D_pad/16, V, 4] in sorted
    order (V = 64 up to 256 dims, else 16)."""
    T, V = ix.tile_size, (64 if ix.D_pad <= 256 else 16)
    cells = ix.sq8_cells.numpy().view(np.uint8)           # [tiles, T/V, G16, V, 16] bytes c ^ 0x80
    assert cells.shape == (ix.total_tiles, T // V, ix.D_pad // 16, V, 16)
    toff = ix.cluster_tile_off.numpy()
    voff = ix.storage.cluster_vec_off.numpy()
    codes = np.zeros((ix.N, ix.D_pad), np.uint8)
    for c in range(ix.nlist):
        li = np.arange(voff[c + 1] - voff[c])
        t, s = toff[c] + li // T, li % T
        codes[voff[c]:voff[c + 1]] = (cells[t, s // V, :, s % V, :] ^ 0x80).reshape(len(li), -1)
    return codes


@pytest.fixture(scope="module")
def wide_ix():
    """D = 300 (D_pad 320 > 256): 16-slot cell blocks, tile 256."""
    xb, xq = datagen.cfg1(N=3000, D=300, B=16, n_centers=8, seed=5)
    ix, cen, lid = build(xb, 6, T=256)
    return ix, xb.numpy(), xq.numpy(), cen, lid


@pytest.mark.parametrize("which", ["hist", "gmm", "wide"])
def test_cells_hold_the_packed_codes(which, hist_ix, gmm_ix, wide_ix):
    """The batched route's 16-byte cells (dims 16 g .. 16 g + 15 of a slot, bytes c ^ 0x80,
    block-major) decode to exactly the codes of sq8_packed, and padded slots hold code 0."""
    ix = {"hist": hist_ix, "gmm": gmm_ix, "wide": wide_ix}[which][0]
    codes, _ = unpack_codes(ix)
    assert np.array_equal(unpack_cells(ix), codes)
    V = 64 if ix.D_pad <= 256 else 16
    cells = ix.sq8_cells.numpy().view(np.uint8)
    pad = ix.tile_orig_ids.numpy() < 0                     # [tiles, T]
    t, s = pad.nonzero()
    assert len(t) > 0
    assert (cells[t, s // V, :, s % V, :] == 0x80).all()
    # one scan block of V slots is one contiguous run of D_pad / 16 * V cells
    assert cells.shape[1:] == (ix.tile_size // V, ix.D_pad // 16, V, 16)


@pytest.mark.parametrize("which", ["hist", "gmm", "wide"])
def test_packing_rebuilt_from_cells(which, hist_ix, gmm_ix, wide_ix):
    """packed_from_cells inverts cells_from_packed bit for bit (narrow and wide cell blocks), so
    an index that releases sq8_packed on the device still saves the reference packing; a
    mutant that forgets the 0x80 flip is caught."""
    from trident_amd.index import packed_from_cells
    ix = {"hist": hist_ix, "gmm": gmm_ix, "wide": wide_ix}[which][0]
    got = packed_from_cells(ix.sq8_cells, ix.D_pad, ix.tile_size)
    assert got.dtype == torch.int32 and torch.equal(got, ix.sq8_packed.view_as(got))
    flip = torch.tensor(-0x7f7f7f80, dtype=torch.int32)
    assert not torch.equal(got ^ flip, ix.sq8_packed.view_as(got))


@pytest.mark.parametrize("which", ["hist", "gmm"])
def test_eps_bounds_quantisation_error(which, hist_ix, gmm_ix):
    ix = (hist_ix if which == "hist" else gmm_ix)[0]
    xr64 = rotated64(ix)
    codes, _ = unpack_codes(ix)
    lid_s = ix.storage.list_ids_sorted.numpy().astype(np.int64)
    vmin = ix.vmin_pad.numpy().astype(np.float64)[lid_s]
    dl = ix.delta_pad.numpy().astype(np.float64)[lid_s]
    xhat = vmin + codes.astype(np.float64) * dl
    err = np.abs(xr64 - xhat)
    eps = ix.eps_pad.numpy().astype(np.float64)[lid_s]
    assert (err <= eps).all()
    # and eps is tight: about half a quantisation step where the dimension has spread
    live = dl > 1e-6
    assert np.median(eps[live] / dl[live]) < 0.51


def test_block_bounds():
    xb, _ = datagen.cfg1(N=600, D=128, B=4, n_centers=4, seed=5)
    ix, _, _ = build(xb, 4, var_block=0)
    assert ix.blk_bounds4.tolist() == [0, 8, 16, 24, 32]
    ix, _, _ = build(xb, 4, var_block=1)
    assert ix.blk_bounds4.tolist() == [0, 4, 8, 16, 24, 32]
    xb, _ = datagen.cfg3(N=700, D=960, B=4, n_centers=4, seed=5)
    ix, _, _ = build(xb, 4, T=256)
    b = ix.blk_bounds4.tolist()
    assert b[0] == 0 and b[-1] == 240 and len(b) == 31 and ix.sq8_packed.shape[2] == 256


def fmaf(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def test_bounds_bracket_distance_cpu_restatement(hist_ix, gmm_ix):
    """float32 numpy restatement of the kernel's dim_params / lb_step / ub_step."""
    for ix, xb, xq, cen, lid in (hist_ix, gmm_ix):
        W = ix.W_combined.numpy().astype(np.float64)
        R = W[:, ix.nlist:ix.nlist + ix.D]
        bvec = ix.b_combined.numpy()[0, ix.nlist:].astype(np.float64)
        codes, _ = unpack_codes(ix)
        voff = ix.storage.cluster_vec_off.numpy()
        xs = ix.storage.xb_sorted.numpy().astype(np.float64)
        rho = (ix.D_pad + 4) * 2.0 ** -24
        lb_scale = ix.rot_sq_max * (1 + rho) * (1 + 1e-12)
        ub_scale = (1 + rho) * (1 + 1e-12) / ix.rot_sq_min
        for qi in range(len(xq)):
            q = xq[qi].astype(np.float64)
            xr = np.zeros(ix.D_pad)
            xr[:ix.D] = q @ R
            xr += bvec
            qe = (ix.D + 3) * 2.0 ** -52 * (np.abs(q[:, None] * np.pad(R, ((0, 0), (0, ix.D_pad - ix.D)))).sum(0) + np.abs(bvec))
            for c in range(0, ix.nlist, 5):
                s, e = voff[c], voff[c + 1]
                if s == e:
                    continue
                vm = ix.vmin_pad.numpy()[c].astype(np.float64)
                dl = ix.delta_pad.numpy()[c]
                ep = ix.eps_pad.numpy()[c].astype(np.float64)
                b64 = vm - xr
                b32 = b64.astype(np.float32)
                E = np.abs(b32.astype(np.float64) - b64) + qe + 2.0 ** -52 * np.abs(b64) + \
                    2.0 ** -24 * (255.0 * dl.astype(np.float64) + np.abs(b32.astype(np.float64))) * (1 + 2.0 ** -20) + 2.0 ** -126
                e32 = ((ep + E) * (1 + 2.0 ** -50)).astype(np.float32)
                e32 = np.where(e32.astype(np.float64) < (ep + E), np.nextafter(e32, np.float32(np.inf)), e32)
                cd = codes[s:e].astype(np.float32)
                a = fmaf(cd, dl[None], b32[None])
                lb = np.zeros(e - s, np.float32)
                ub = np.zeros(e - s, np.float32)
                for d in range(ix.D_pad):
                    l = np.maximum(np.abs(a[:, d]) - e32[d], np.float32(0))
                    lb = fmaf(l, l, lb)
                    u = np.abs(a[:, d]) + e32[d]
                    ub = fmaf(u, u, ub)
                d64 = ((xs[s:e] - q) ** 2).sum(1)
                assert (lb.astype(np.float64) / lb_scale <= d64 * (1 + 1e-12)).all()
                assert (ub.astype(np.float64) * ub_scale >= d64 * (1 - 1e-12)).all()


def test_centroid_band_layouts_positions():
    """The matrix-core tile layout of the centroids: float4 (t Dq/16 + j) 64 + l holds dims
    (l / 16) Dq/4 + 4 j .. + 3 of centroid 16 t + l % 16 (zero past D and past nlist)."""
    from trident_amd import ext as E
    g = torch.Generator().manual_seed(5)
    for D, nlist in ((96, 40), (128, 64), (20, 17)):
        W = torch.randn((D, nlist + 32), generator=g)
        rows, tiles, norms, nmax = E.centroid_band_layouts(W, nlist)
        Dq = E.band_dq(D)
        S = Dq // 4
        cen = (-0.5 * W[:, :nlist]).t()
        assert torch.equal(rows[:, :D], cen) and not rows[:, D:].any()
        t4 = tiles.view(-1, 4)
        for c in range(0, (nlist + 15) // 16 * 16, 3):
            for d in range(0, Dq, 5):
                gq, sd = divmod(d, S)
                f = ((c // 16) * (S // 4) + sd // 4) * 64 + (c % 16) + 16 * gq
                want = float(cen[c, d]) if c < nlist and d < D else 0.0
                assert float(t4[f, sd % 4]) == want, (D, nlist, c, d)
        n64 = (cen.double() ** 2).sum(1)  # summation order may differ in the last bit
        assert torch.allclose(norms.double(), n64, rtol=1e-6, atol=0)
        assert abs(nmax - float(n64.max())) <= 1e-12 * float(n64.max())


@pytest.mark.parametrize("which", ["hist", "gmm"])
def test_derived_vec_ar_matches_the_builder(which, hist_ix, gmm_ix):
    """index.derive_vec_Ar (the drop-in path for an index passed in the reference layout alone)
    recomputes the builder's per-vector scalars from sq8_packed, the stored rotation and the
    base: identical bits, and r bounds |x R + b - x_hat| measured independently in numpy."""
    from trident_amd.index import cells_from_packed, derive_vec_Ar
    ix = (hist_ix if which == "hist" else gmm_ix)[0]
    st = ix.storage
    got = derive_vec_Ar(ix.sq8_packed, st.cluster_vec_off, ix.cluster_tile_off, st.xb_sorted, ix.W_combined,
                        ix.b_combined, ix.vmin_pad, ix.delta_pad, ix.per_cluster_sq8, ix.nlist, ix.tile_size)
    assert torch.equal(got, ix.vec_Ar)
    assert torch.equal(cells_from_packed(ix.sq8_packed, ix.D_pad, ix.tile_size), ix.sq8_cells)
    # independent check of r on every vector: decode the codes from the cells, rotate in numpy
    D, Dp, nl = ix.D, ix.D_pad, ix.nlist
    R = ix.W_combined[:, nl:nl + D].double().numpy()
    b = ix.b_combined.reshape(-1)[nl:nl + D].double().numpy()
    xb = st.xb_sorted.double().numpy()
    vo = st.cluster_vec_off.numpy()
    lid = np.repeat(np.arange(nl), np.diff(vo))
    packed = ix.sq8_packed.numpy().reshape(-1, Dp // 4, ix.tile_size)
    to = ix.cluster_tile_off.numpy()
    loc = np.arange(len(xb)) - vo[lid]
    codes = packed[to[lid] + loc // ix.tile_size, :, loc % ix.tile_size].view(np.uint8).astype(np.float64)
    xhat = ix.vmin_pad.double().numpy()[lid] + codes * ix.delta_pad.double().numpy()[lid]
    xr = np.zeros_like(xhat)
    xr[:, :D] = xb @ R + b
    r_np = np.sqrt(((xr - xhat) ** 2).sum(1))
    assert (got[:, 1].double().numpy() >= r_np).all()
    a_np = ((codes * ix.delta_pad.double().numpy()[lid]) ** 2).sum(1)
    assert (got[:, 0].double().numpy() <= a_np).all()


def test_tile_band_brackets_residual_norms(hist_ix):
    """tile_r_minmax holds, per tile, float32 bounds around every |x - c(x)| of its vectors."""
    ix, xb, _, cen, lid = hist_ix
    st = ix.storage
    T, nl = ix.tile_size, ix.nlist
    vo = st.cluster_vec_off.numpy()
    to = ix.cluster_tile_off.numpy()
    xs = st.xb_sorted.double().numpy()
    lids = np.repeat(np.arange(nl), np.diff(vo))
    r = np.sqrt(((xs - ix.centroids.double().numpy()[lids]) ** 2).sum(1))
    tile = to[lids] + (np.arange(len(xs)) - vo[lids]) // T
    band = ix.tile_r_minmax.double().numpy()
    assert (band[tile, 0] <= r).all() and (band[tile, 1] >= r).all()
    # tight: the band of each tile is within float32 rounding of its extreme norms
    for t in np.unique(tile)[:50]:
        rr = r[tile == t]
        assert band[t, 0] >= rr.min() * (1 - 1e-6) and band[t, 1] <= rr.max() * (1 + 1e-6)


def test_fine_codes_bound_the_rotated_rows():
    """Fine level: per row, codes are rint((x_rot - offset) / step) in 16 bits with offset <= the
    row's smallest coordinate and step >= its range / 65535, and rho bounds |x_rot - x_fine| for
    every row (float64 rotation of the stored float32 map)."""
    xb, _ = datagen.cfg1(N=3000, D=40, B=4, n_centers=8, seed=5)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, 12, seed=0, niter=4)
    st = SharedClusterStorage(xb.numpy(), lid, r, 12, device="cpu")
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device="cpu", max_batch=8, max_nprobe=8,
                        fine_level=True)
    assert ix.fine_codes.shape == (3000, ix.D_pad) and ix.fine_codes.dtype == torch.int16
    D, Dp, nl = ix.D, ix.D_pad, ix.nlist
    R = ix.W_combined[:, nl:nl + D].double().numpy()
    bb = ix.b_combined.reshape(-1)[nl:nl + D].double().numpy()
    x = st.xb_sorted.double().numpy()
    xr = np.zeros((len(x), Dp))
    xr[:, :D] = x @ R + bb
    qp = ix.fine_qp.double().numpy()
    off, step, rho = qp[:, :1], qp[:, 1:2], qp[:, 2]
    assert (off[:, 0] <= xr.min(1)).all() and (step[:, 0] * 65535 >= xr.max(1) - off[:, 0]).all()
    codes = ix.fine_codes.numpy().astype(np.int64) & 0xFFFF
    assert np.array_equal(codes, np.clip(np.rint((xr - off) / step), 0, 65535))
    xf = off + codes * step
    err = np.sqrt(((xr - xf) ** 2).sum(1))
    assert (err <= rho).all()
    # 16 bits per dimension: far below the SQ8 residual norm
    r1 = ix.vec_Ar[:, 1].double().numpy()
    assert np.median(rho / r1) < 0.05



@pytest.mark.parametrize("which", ["hist", "gmm", "wide"])
def test_row_code_norms(which, hist_ix, gmm_ix, wide_ix):
    """vec_cn: per sorted row, sqrt(sum (code - 128)^2) over D_pad dims rounded up to float32 --
    checked against the codes unpacked from sq8_packed (the reference tile packing, not the
    cells the norms are computed from) with an exact integer sum; and the Cauchy-Schwarz bound
    it feeds (|sum (code - 128) lo| <= cn |lo|) against random int8 lo planes."""
    ix = {"hist": hist_ix, "gmm": gmm_ix, "wide": wide_ix}[which][0]
    st = ix.storage
    T, D_pad = ix.tile_size, ix.D_pad
    vec_off = st.cluster_vec_off.long().numpy()
    tile_off = ix.cluster_tile_off.long().numpy()
    packed = ix.sq8_packed.view(torch.uint8).reshape(-1, D_pad // 4, T, 4).numpy()
    cn = ix.vec_cn.numpy()
    assert cn.dtype == np.float32 and cn.shape == (st.N,)
    rng = np.random.default_rng(3)
    for c in range(ix.nlist):
        loc = np.arange(vec_off[c + 1] - vec_off[c])
        codes = packed[tile_off[c] + loc // T, :, loc % T, :].reshape(len(loc), -1).astype(np.int64)
        ssq = ((codes - 128) ** 2).sum(1)
        got = cn[vec_off[c]:vec_off[c + 1]].astype(np.float64)
        assert np.all(got ** 2 >= ssq)                                        # upper bounds
        # at most one float32 step above the least upper bound (the 2^-50 raise before rounding
        # moves exact squares up by one step)
        z = np.float32(0)
        below2 = np.nextafter(np.nextafter(cn[vec_off[c]:vec_off[c + 1]], z), z).astype(np.float64)
        assert np.all((below2 ** 2 < ssq) | (ssq == 0))
        lo = rng.integers(-128, 128, size=(len(loc), D_pad))
        dots = np.abs(((codes - 128) * lo).sum(1)).astype(np.float64)
        assert np.all(dots <= got * np.sqrt((lo * lo).sum(1).astype(np.float64)))


def _two_shapes(seed=0):
    """Blob clusters (isotropic Gaussians, 32 dims) and elongated ones (a uniform segment per
    cluster with small noise), 12 clusters of 4,000 rows each, with each cluster's mean."""
    g = np.random.default_rng(seed)
    n, k, D = 4000, 12, 32
    lid = np.repeat(np.arange(k), n).astype(np.int64)
    centers = g.uniform(0, 100, size=(k, D)).astype(np.float32)
    blob = centers[lid] + g.normal(0, 4.0, size=(n * k, D)).astype(np.float32)
    direction = g.normal(size=(k, D)).astype(np.float32)
    direction /= np.linalg.norm(direction, axis=1, keepdims=True)
    t = g.uniform(-30, 30, size=(n * k, 1)).astype(np.float32)
    line = centers[lid] + t * direction[lid] + g.normal(0, 0.05, size=(n * k, D)).astype(np.float32)
    out = {}
    for name, x in (("blob", blob), ("line", line)):
        mean = np.stack([x[lid == c].mean(0) for c in range(k)])
        r = np.linalg.norm(x - mean[lid], axis=1).astype(np.float32)
        out[name] = (x, lid, r, k)
    return out


def test_within_cluster_order_follows_the_seeding_score():
    """Rows ordered by residual norm seed tighter thresholds on blob clusters (the first slice is
    the core, near every query of the cluster) and far looser ones on elongated clusters (the
    core is far from a query at either end); 'auto' takes the better order, and either order is
    a cluster-sorted permutation with the same clusters."""
    from trident_amd.index import seed_order_scores
    sets = _two_shapes()
    for name, (x, lid, r, k) in sets.items():
        sc = seed_order_scores(torch.as_tensor(x), torch.as_tensor(lid), torch.as_tensor(r), k, sv=1024)
        if name == "blob":
            assert sc["residual"] < 0.99 * sc["id"], sc
        else:
            assert sc["id"] < 0.99 * sc["residual"], sc
    for name, (x, lid, r, k) in sets.items():
        st = {w: SharedClusterStorage(x, lid, r, k, device="cpu", within=w) for w in ("id", "residual")}
        for w, s in st.items():
            perm = s.sort_perm.astype(np.int64)
            assert np.array_equal(np.sort(perm), np.arange(len(lid)))
            assert np.all(np.diff(lid[perm]) >= 0)
            np.testing.assert_array_equal(s.cluster_vec_off.cpu().numpy(), st["id"].cluster_vec_off.cpu().numpy())
            np.testing.assert_array_equal(s.xb_sorted.cpu().numpy(), x[perm])
        pr = st["residual"].sort_perm.astype(np.int64)
        for c in range(k):
            rc = r[pr[lid[pr] == c]]
            assert np.all(np.diff(rc) >= 0)
        assert np.array_equal(st["id"].sort_perm, np.argsort(lid, kind="stable").astype(np.int32))
        assert SharedClusterStorage(x, lid, r, k, device="cpu").within == ("residual" if name == "blob" else "id")
