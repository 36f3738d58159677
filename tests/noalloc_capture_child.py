"""Child process of tests/test_streams_graph_gpu.py: the process's FIRST call of
tilemix_tiles_importance_noalloc is made while torch captures a CUDA graph, so
the library looks up its scratch array's device address during the capture.
The graph is then replayed three times, between eager work, and every replay's
tile codes are compared with the workspace entry point's. Prints one line
ending in OK and exits 0 on success."""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tilemix-cuda_amd"))


def main() -> int:
    import torch
    import tilemix as tm

    heads, M, N, d, tr, tk, fraction = 2, 1024, 1536, 64, 128, 64, 0.25
    print(f"noalloc capture child: heads={heads} M={M} N={N} d={d} tile={tr}x{tk}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    q = torch.randn(heads, M, d, generator=g, device="cuda")
    k = torch.randn(heads, N, d, generator=g, device="cuda")
    q[..., :2] *= 8.0
    k[..., :2] *= 8.0
    q, k = q.half().contiguous(), k.half().contiguous()
    tiles = (heads, (M + tr - 1) // tr, (N + tk - 1) // tk)
    need = tm.importance_workspace_bytes(heads, M, N, tr, tk)
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    expected = torch.full(tiles, 0xEE, dtype=torch.uint8, device="cuda")
    tm.check(tm.tiles_importance(q, k, heads, M, N, d, tr, tk, fraction, ws, need, expected), "importance")
    torch.cuda.synchronize()

    codes = torch.full(tiles, 0xEE, dtype=torch.uint8, device="cuda")
    graph = torch.cuda.CUDAGraph()
    print("noalloc capture child: first noalloc call inside the capture", flush=True)
    with torch.cuda.graph(graph):
        rc = tm.tiles_importance_noalloc(q, k, heads, M, N, d, tr, tk, fraction, codes)
    tm.check(rc, "noalloc importance under capture")
    torch.cuda.synchronize()
    for replay in range(3):
        codes.fill_(0xEE)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(codes, expected):
            print(f"noalloc capture child: replay {replay} differs from the workspace entry point", flush=True)
            return 1
    print("noalloc capture child: 3 replays equal the workspace entry point: OK", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
