import sys, ctypes
sys.path.insert(0, '/root/repo/speculative-decoder_amd'); sys.path.insert(0, '/root/repo'); sys.path.insert(0, '/root/repo/tests/golden')
import torch
import bench
lib = ctypes.CDLL('/root/repo/_work/exp/libtilefloor.so')
lib.tile_floor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
dev = torch.device('cuda', 0)
POOL = 1 << 30  # 1 GiB pool per buffer
NB = 3
bufs = [torch.empty(POOL // 4, dtype=torch.int32, device=dev).random_() for _ in range(NB)]
out = torch.zeros(65536, device=dev)
st = lambda: torch.cuda.current_stream().cuda_stream
total = 269_000_000
for tile_bytes in (2048, 4096, 16384, 65536):
    n_tiles = POOL // tile_bytes
    tiles = total // tile_bytes
    idx = torch.randperm(n_tiles, device=dev)[:tiles].to(torch.int32).contiguous()
    for per_wg_bytes in (65536, 131072):
        tiles_per_wg = per_wg_bytes // tile_bytes
        wgs = tiles // tiles_per_wg
        it = [0]
        def f():
            b = bufs[it[0] % NB]; it[0] += 1
            assert lib.tile_floor(b.data_ptr(), idx.data_ptr(), out.data_ptr(), wgs, tiles_per_wg, tile_bytes, tiles, st()) == 0
        f(); torch.cuda.synchronize()
        us = bench.graph_time_us(f, per_graph=NB * 4, replays=5)
        nb = wgs * tiles_per_wg * tile_bytes
        print(f'random {tile_bytes}-byte tiles, {per_wg_bytes//1024} KB per WG, {nb/1e6:.0f} MB: {us:.2f} us {nb/us/1e3:.0f} GB/s', flush=True)
