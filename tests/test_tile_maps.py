"""The integer maps of the GEMM kernels (rust-gpu_amd/csrc/kernels/tile_map.h),
compiled for the host from the same source and run over whole index ranges
on the CPU, after the reference's CPU memory-safety simulation
(tests/gemm_memory_safety.rs:25-228: load coverage and bounds, LDS address
bijection, store coverage):

- the workgroup -> XCD remap and the grouped tile order are bijections, so
  every output tile is computed exactly once;
- for every GEMM instance of gemm_bf16.hip, the global -> LDS DMA map of a
  stage writes each (row, 16-byte k chunk) of the A and B tiles exactly
  once, and every MFMA operand read finds in LDS the row and chunk it
  expects, under the XOR swizzles (row-major A / NT B, and the NN B tile's
  transposed-read layout); the map is restated from gemm_bf16.hip
  (TileLoader and the ping-pong split), the swizzles are the compiled ones."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KDIR = os.path.join(ROOT, "rust-gpu_amd", "csrc", "kernels")

WRAP = r"""
#include "tile_map.h"
extern "C" {
uint32_t swz_rows_c(int ch, uint32_t r) {
    switch (ch) {
    case 2: return t0::swz_rows<2>(r);
    case 4: return t0::swz_rows<4>(r);
    case 8: return t0::swz_rows<8>(r);
    case 16: return t0::swz_rows<16>(r);
    case 32: return t0::swz_rows<32>(r);
    }
    return ~0u;
}
uint32_t swz_nn_c(int chb, uint32_t r) {
    switch (chb) {
    case 4: return t0::swz_nn<4>(r);
    case 8: return t0::swz_nn<8>(r);
    case 16: return t0::swz_nn<16>(r);
    case 32: return t0::swz_nn<32>(r);
    case 64: return t0::swz_nn<64>(r);
    }
    return ~0u;
}
void xcd_remap_all(uint32_t total, uint32_t* out) {
    for (uint32_t b = 0; b < total; b++) out[b] = t0::xcd_remap(b, total);
}
void grouped_all(uint32_t tiles_m, uint32_t tiles_n, uint32_t group_m, uint32_t* tm, uint32_t* tn) {
    for (uint32_t id = 0; id < tiles_m * tiles_n; id++) t0::grouped_tile(id, tiles_m, tiles_n, group_m, tm[id], tn[id]);
}
}
"""


@pytest.fixture(scope="module")
def maps(tmp_path_factory):
    d = tmp_path_factory.mktemp("tile_maps")
    src, so = d / "wrap.cpp", d / "libmaps.so"
    src.write_text(WRAP)
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-shared", "-fPIC", "-I", KDIR, "-o", str(so),
                    str(src)], check=True)
    lib = C.CDLL(str(so))
    for f in ("swz_rows_c", "swz_nn_c"):
        getattr(lib, f).argtypes = [C.c_int, C.c_uint32]
        getattr(lib, f).restype = C.c_uint32
    lib.xcd_remap_all.argtypes = [C.c_uint32, C.POINTER(C.c_uint32)]
    lib.grouped_all.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
    return lib


def instances():
    """(BM, BN, BK, WM, WN, STAGES) of every T0_GEMM_BOTH / T0_GEMM_VG_BOTH line."""
    text = open(os.path.join(KDIR, "gemm_bf16.hip")).read()
    found = re.findall(r"^T0_GEMM(?:_VG)?_BOTH\((\d+), (\d+), (\d+), (\d+), (\d+), (\d+)", text, flags=re.M)
    assert len(found) >= 20
    return sorted({tuple(int(x) for x in f) for f in found})


def test_xcd_remap_is_a_bijection_with_contiguous_xcd_ranges(maps):
    for total in list(range(1, 1100)) + [4095, 4096, 4097, 16384, 65535]:
        out = (C.c_uint32 * total)()
        maps.xcd_remap_all(total, out)
        got = list(out)
        assert sorted(got) == list(range(total)), total
        for x in range(8):   # workgroups of one XCD (b % 8 == x) own one contiguous range
            ids = sorted(got[x::8])
            assert ids == list(range(ids[0], ids[0] + len(ids))) if ids else True, (total, x)


def test_grouped_tile_order_covers_the_grid_once(maps):
    for tiles_m in range(1, 41):
        for tiles_n in (1, 2, 3, 7, 16, 33):
            for group_m in (1, 2, 4, 8):
                n = tiles_m * tiles_n
                tm, tn = (C.c_uint32 * n)(), (C.c_uint32 * n)()
                maps.grouped_all(tiles_m, tiles_n, group_m, tm, tn)
                cells = sorted(zip(tm, tn))
                assert cells == [(i, j) for i in range(tiles_m) for j in range(tiles_n)], (tiles_m, tiles_n, group_m)


@pytest.mark.parametrize("ch", [2, 4, 8, 16, 32])
def test_row_swizzle_range_and_period(maps, ch):
    """Chunk indices stay inside the row, and a row's swizzle depends on
    the row mod 32 only: the operand reads take it from lane & 31 for rows
    that lie whole multiples of 32 further on."""
    for r in range(4096):
        v = maps.swz_rows_c(ch, r)
        assert v < ch and v == maps.swz_rows_c(ch, r % 32), (ch, r)


def _row_tile(maps, rows, bk, chunks_pos):
    """LDS 16-byte slot -> (row, k chunk) for the positions DMA'd: a row-major
    [rows][bk] bf16 tile, chunk c of row r stored at slot r * CH + (c ^ swz(r))."""
    ch = bk // 8
    held = {}
    for pos in chunks_pos:
        r, s = pos // (bk * 2), (pos % (bk * 2)) // 16
        c = s ^ maps.swz_rows_c(ch, r)
        assert r < rows and c < ch
        assert pos // 16 not in held
        held[pos // 16] = (r, c)
    assert sorted(held.values()) == [(r, c) for r in range(rows) for c in range(ch)]
    return held


def _nn_tile(maps, bk, bn, chunks_pos):
    chb = bn // 8
    held = {}
    for pos in chunks_pos:
        r, s = pos // (bn * 2), (pos % (bn * 2)) // 16
        c = s ^ maps.swz_nn_c(chb, r)
        assert r < bk and c < chb
        assert pos // 16 not in held
        held[pos // 16] = (r, c)
    assert sorted(held.values()) == [(r, c) for r in range(bk) for c in range(chb)]
    return held


def _positions(nw, loads):
    """TileLoader: wave w's load j covers bytes (w * loads + j) * 1 KiB + lane * 16."""
    return [(w * loads + j) * 1024 + lane * 16 for w in range(nw) for j in range(loads) for lane in range(64)]


@pytest.mark.parametrize("inst", instances(), ids=lambda t: "{}x{}x{}_w{}x{}_s{}".format(*t))
def test_gemm_stage_maps_write_once_and_reads_find_their_chunks(maps, inst):
    bm, bn, bk, wm, wn, stages = inst
    nw, tm, tn = wm * wn, bm // wm, bn // wn
    fm, fn = tm // 32, tn // 32
    a_bytes, b_bytes = bm * bk * 2, bn * bk * 2
    a_loads, b_loads = a_bytes // (1024 * nw), b_bytes // (1024 * nw)
    assert a_loads * 1024 * nw == a_bytes and b_loads * 1024 * nw == b_bytes
    pos_a, pos_b = _positions(nw, a_loads), _positions(nw, b_loads)
    if bm == 256 and bn == 256 and bk == 32 and nw == 8 and stages == 4 and wm == 2:
        # the ping-pong split: waves 0-3 DMA the A tile, waves 4-7 the B tile,
        # four 1 KiB chunks each (q = (wave & 3) * 4 + j)
        pp = [((w & 3) * 4 + j) * 1024 + lane * 16 for w in range(4) for j in range(4) for lane in range(64)]
        assert sorted(pp) == sorted(pos_a) == sorted(pos_b)
    a = _row_tile(maps, bm, bk, pos_a)
    bt = _row_tile(maps, bn, bk, pos_b)          # NT: B is WT[n][k]
    bnn = _nn_tile(maps, bk, bn, pos_b)          # NN: B[k][n]
    cha, chb = bk // 8, bn // 8
    for w in range(nw):
        wmi, wni = w // wn, w % wn
        for lane in range(64):
            l32, hi = lane & 31, lane >> 5
            sw = maps.swz_rows_c(cha, l32)
            for kk in range(bk // 16):
                for i in range(fm):
                    addr = (wmi * tm + l32) * (bk * 2) + (((kk * 2 + hi) ^ sw) * 16) + i * 32 * (bk * 2)
                    assert a[addr // 16] == (wmi * tm + l32 + 32 * i, kk * 2 + hi), (inst, w, lane, kk, i)
                for j in range(fn):
                    addr = (wni * tn + l32) * (bk * 2) + (((kk * 2 + hi) ^ sw) * 16) + j * 32 * (bk * 2)
                    assert bt[addr // 16] == (wni * tn + l32 + 32 * j, kk * 2 + hi), (inst, w, lane, kk, j)
            # NN: each 16-lane group reads 4 k rows x 2 chunks per 32 columns
            # (ds_read_b64_tr_b16 at k rows r and r + 4); the chunk a lane
            # addresses must hold its k row and column chunk
            g, i16 = lane >> 4, lane & 15
            s = maps.swz_nn_c(chb, i16 >> 2)
            row0 = (g >> 1) * 8 + (i16 >> 2)
            for j in range(fn):
                c16 = (wni * tn + j * 32) // 8 + (g & 1) * 2 + (i16 & 3) // 2
                col = row0 * (bn * 2) + ((c16 ^ s) * 16) + (i16 & 1) * 8
                for kk in range(bk // 16):
                    for dr in (0, 4):
                        p0 = col + kk * 16 * (bn * 2) + dr * (bn * 2)
                        assert bnn[p0 // 16] == (row0 + kk * 16 + dr, c16), (inst, w, lane, j, kk, dr)
