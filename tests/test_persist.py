"""save / load in the reference's on-disk format "MAIVS2\\0\\1" (src/persist.rs:28-281).

The reference's own checks (tests/test_index.py:184-217, 490-512) are restated here: n_live,
quant_scale and the cell count survive a reload; deleted ids stay deleted; with no mutation in
between, save -> load (-> set_fastscan(True); compact()) is an identity. The byte layout is pinned
by an independent reader written from src/persist.rs:145-199, which must consume exactly the
reference's blocks and stop at this library's extension trailer. A file without the trailer (what
the reference writes) loads with the reference's defaults.
"""
import os
import struct

import numpy as np
import pytest

import maivs_amd as M

from .conftest import small_clustered

MAGIC = b"MAIVS2\x00\x01"
TRAILER = b"MAIVSX\x00\x01"


def _read_reference_layout(path):
    """The reference's load_index (src/persist.rs:145-199), field by field, with numpy.
    Returns (header, floats, blocks, cells, offset where the reference stops reading)."""
    buf = open(path, "rb").read()
    assert buf[:8] == MAGIC
    off = 8
    hdr = struct.unpack_from("<16Q", buf, off)
    off += 128
    floats = struct.unpack_from("<4f", buf, off)
    off += 16

    def pod(dtype):
        nonlocal off
        (n,) = struct.unpack_from("<Q", buf, off)
        off += 8
        a = np.frombuffer(buf, dtype=dtype, count=n, offset=off).copy()
        off += n * np.dtype(dtype).itemsize
        return a

    names = [("bits", "<u8"), ("scan_i8", "i1"), ("rr_f16", "<u2"), ("sq_min", "<f4"), ("sq_step", "<f4"),
             ("vecs_f32", "<f4"), ("ext_ids", "<u8"), ("slot_cell", "<u4"), ("free_slots", "<u4"),
             ("slot_cells", "<u4"), ("tags", "<u4")]
    blocks = {n: pod(t) for n, t in names}
    (ncell,) = struct.unpack_from("<Q", buf, off)
    off += 8
    cells = []
    for _ in range(ncell):
        members, s, cent = pod("<u4"), pod("<f4"), pod("<f4")
        rb, rm = struct.unpack_from("<2f", buf, off)
        off += 8
        cells.append((members, s, cent, rb, rm))
    return hdr, floats, blocks, cells, off, buf


@pytest.fixture(scope="module")
def small_index():
    x = small_clustered(6000, 64, 48, seed=3)
    ix = M.preset(64, len(x))
    ix.train_centroids(x, 47)
    ix.add_batch(list(range(1000, 1000 + len(x))), x)
    ix.compact()
    return ix, x


def test_roundtrip_is_identity(small_index, tmp_path):
    ix, _ = small_index
    p = str(tmp_path / "idx.maivs")
    ix.save(p)
    ix2 = M.FlatCellIndex.load(p)
    assert len(ix2) == len(ix)
    s1, s2 = ix.stats(), ix2.stats()
    assert abs(s1["quant_scale"] - s2["quant_scale"]) < 1e-9
    assert s1["n_cells"] == s2["n_cells"]
    # the trailer restores FastScan and compaction: the arena is ready for the GPU without a rebuild
    assert ix2.cellmajor_blocker(True) == ""
    a, b = ix._arena_arrays(), ix2._arena_arrays()
    assert a.keys() == b.keys()
    for key in a:
        if isinstance(a[key], np.ndarray):
            assert np.array_equal(a[key], b[key]), key
        else:
            assert a[key] == b[key], key
    assert np.array_equal(ix._ext_ids(), ix2._ext_ids())
    assert np.array_equal(ix._codes(), ix2._codes())
    assert ix._search_params(10, 16) == ix2._search_params(10, 16)


def test_file_layout_is_the_reference_format(small_index, tmp_path):
    ix, x = small_index
    p = str(tmp_path / "idx.maivs")
    ix.save(p)
    hdr, floats, blk, cells, end, buf = _read_reference_layout(p)
    n = len(x)
    a = ix._arena_arrays()
    # header: dim, scan_mode binary = 2, rerank_factor, dim_pad, n_words, seed, n_live, max_assign,
    # shortlist_mult, i8_rerank, keep_f32, adaptive, two_stage, tree_route, tree_min_cells, tree_fanout
    assert hdr == (64, 2, 32, 64, 1, 0x5EED, n, 2, 2, 0, 1, 1, 1, 1, 2048, 16)
    assert floats[2] == pytest.approx(0.02)  # at_margin
    assert np.array_equal(blk["ext_ids"], ix._ext_ids())
    assert np.array_equal(blk["bits"], ix._codes())
    assert np.array_equal(blk["vecs_f32"].reshape(n, 64), a["vecs_f32"].reshape(n, 64))
    assert np.array_equal(blk["slot_cells"], a["slot_cells"])
    assert len(blk["rr_f16"]) == 0 and len(blk["scan_i8"]) == 0 and len(blk["tags"]) == 0
    assert len(cells) == a["n_cells"]
    mem = np.concatenate([c[0] for c in cells])
    assert np.array_equal(mem, a["members"])
    cent = np.stack([c[2] for c in cells])
    assert np.array_equal(cent.reshape(-1), a["centroids"])
    assert np.array_equal(np.array([c[3] for c in cells], np.float32), a["r_bound"])
    # the reference stops here; the rest is this library's trailer
    assert buf[end:end + 8] == TRAILER
    (nf,) = struct.unpack_from("<Q", buf, end + 8)
    assert len(buf) == end + 16 + 8 * nf
    fields = struct.unpack_from(f"<{nf}Q", buf, end + 16)
    assert fields[0] == 1 and fields[1] == 1  # fastscan, compacted
    assert struct.unpack("<f", struct.pack("<I", fields[7]))[0] == 1.0  # orthogonal-polysemy strength


def test_reference_written_file_loads_with_its_defaults(small_index, tmp_path):
    """A file without the trailer is what the reference writes. It loads with FastScan off and
    uncompacted (src/persist.rs:265-271); set_fastscan(True); compact() then gives back the same
    arena (the reference's 'FastScan save/load/compact is an identity', tests/test_index.py:504-512)."""
    ix, _ = small_index
    p = str(tmp_path / "idx.maivs")
    ix.save(p)
    *_, end, buf = _read_reference_layout(p)
    q = str(tmp_path / "ref.maivs")
    with open(q, "wb") as f:
        f.write(buf[:end])
    ix2 = M.FlatCellIndex.load(q)
    assert "not compacted" in ix2.cellmajor_blocker(True)
    ix2.set_fastscan(True)
    ix2.compact()
    assert ix2.cellmajor_blocker(True) == ""
    a, b = ix._arena_arrays(), ix2._arena_arrays()
    for key in ("fs_codes", "fs_off", "mem_off", "members", "slot_cells", "cent_bits", "cent_sq8", "r_bound"):
        assert np.array_equal(a[key], b[key]), key


def test_deleted_ids_stay_deleted(tmp_path):
    """tests/test_index.py:213-222: n_live and the deletions survive a reload."""
    x = small_clustered(3000, 32, 24, seed=5)
    ix = M.preset(32, len(x))
    ix.train_centroids(x, 23)
    ix.add_batch(list(range(len(x))), x)
    victims = np.random.RandomState(1).choice(len(x), 300, replace=False)
    for v in victims:
        assert ix.remove(int(v))
    p = str(tmp_path / "d.maivs")
    ix.save(p)  # uncompacted: free slots still hold stale ids
    ixl = M.FlatCellIndex.load(p)
    assert len(ixl) == len(x) - 300
    for v in victims[:20]:
        assert ixl.remove(int(v)) is False
    assert ixl.remove(int(np.setdiff1d(np.arange(len(x)), victims)[0])) is True
    ixl.compact()
    ids = set(ixl._ext_ids().tolist())
    assert not ids & set(victims.tolist())


def test_tags_travel_with_the_file(small_index, tmp_path):
    x = small_clustered(2000, 32, 16, seed=9)
    ix = M.preset(32, len(x))
    ix.train_centroids(x, 15)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    tags = np.random.RandomState(2).randint(0, 1000, len(x))
    ix.set_tags(list(range(len(x))), [int(t) for t in tags])
    p = str(tmp_path / "t.maivs")
    ix.save(p)
    _, _, blk, _, _, _ = _read_reference_layout(p)
    ext = ix._ext_ids()
    assert np.array_equal(blk["tags"], tags[ext].astype(np.uint32))


def test_bad_files_raise(tmp_path, small_index):
    ix, _ = small_index
    bad = tmp_path / "bad.maivs"
    bad.write_bytes(b"MAIVS2\x00\x02" + b"\x00" * 200)
    with pytest.raises(ValueError, match="bad magic or format version"):
        M.FlatCellIndex.load(str(bad))
    with pytest.raises(OSError):
        M.FlatCellIndex.load(str(tmp_path / "missing.maivs"))
    p = str(tmp_path / "idx.maivs")
    ix.save(p)
    whole = open(p, "rb").read()
    for cut in (20, 200, len(whole) // 2, len(whole) - 200):
        t = tmp_path / f"trunc{cut}.maivs"
        t.write_bytes(whole[:cut])
        with pytest.raises((OSError, ValueError)):
            M.FlatCellIndex.load(str(t))
    # a member index past the slot count is refused before anything reaches the GPU
    *_, end, buf = _read_reference_layout(p)
    b = bytearray(buf)
    hdr_end = 8 + 128 + 16
    off = hdr_end
    for itemsize in (8, 1, 2, 4, 4, 4, 8, 4, 4, 4, 4):
        (n,) = struct.unpack_from("<Q", b, off)
        off += 8 + n * itemsize
    off += 8  # n_cells
    (nm,) = struct.unpack_from("<Q", b, off)
    assert nm > 0
    struct.pack_into("<I", b, off + 8, 0xFFFFFFF0)
    c = tmp_path / "corrupt.maivs"
    c.write_bytes(bytes(b))
    with pytest.raises(ValueError, match="corrupt index file"):
        M.FlatCellIndex.load(str(c))


@pytest.mark.gpu
def test_search_identical_after_reload(quality50k, mix50k, tmp_path):
    """tests/test_index.py:184-193: search results identical after reload, here on the GPU."""
    _, queries, _ = mix50k
    q = np.ascontiguousarray(queries[:500])
    ids1, sc1 = quality50k.search_batch(q, 10, 16, 1.0, 8.0, True)
    p = str(tmp_path / "q50k.maivs")
    quality50k.save(p)
    ix2 = M.FlatCellIndex.load(p)
    ids2, sc2 = ix2.search_batch(q, 10, 16, 1.0, 8.0, True)
    assert ids1 == ids2
    assert np.array_equal(np.array(sc1, np.float32), np.array(sc2, np.float32))
    os.remove(p)
