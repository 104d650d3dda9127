"""Per-sample sums over a packed upper triangle held in a torch tensor
(test infrastructure; the full-size GPU tests run it on the device, the CPU
tests pin it against a plain numpy loop)."""


def tri_start(n, i):
    return i * n - i * (i - 1) // 2


def symmetric_row_sums(u, n, block=256):
    """u: 1-D integer tensor, the packed upper triangle of an n x n
    symmetric matrix (row i holds columns i..n-1).  Returns an int64 tensor
    of n per-sample sums over row i and column i, the diagonal taken from
    each side (it is 0 for co-occurrence counts)."""
    import torch

    dev = u.device
    out = torch.zeros(n, dtype=torch.int64, device=dev)
    for r0 in range(0, n, block):
        r1 = min(n, r0 + block)
        e0, e1 = tri_start(n, r0), tri_start(n, r1)
        seg = u[e0:e1].to(torch.int64)
        rows = torch.arange(r0, r1, device=dev)
        lens = n - rows  # entries of row i: columns i..n-1
        starts = torch.cumsum(lens, 0) - lens  # first entry of each row in seg
        # row parts from a running sum (no atomics on one address per row)
        cs = torch.cumsum(seg, 0)
        prev = torch.where(starts > 0, cs[(starts - 1).clamp(min=0)], torch.zeros_like(starts))
        out[r0:r1] += cs[starts + lens - 1] - prev
        # column parts: entry k of the block is column k - starts[row] + row
        rid = torch.repeat_interleave(rows, lens, output_size=e1 - e0)
        col = torch.arange(e1 - e0, device=dev) - starts[rid - r0] + rid
        out.index_add_(0, col, seg)
    return out
