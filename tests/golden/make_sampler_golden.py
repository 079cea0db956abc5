"""Writes tests/golden/sampler_rand.npz: Triton's own generator outputs, the
noise source of the reference's Gumbel-max sampler
(kernels/fused_sampler_ops.py:67, `u = tl.rand(seed + row, offs)`).

Triton (a dependency of the reference; triton 3.6.0 in this image) is run in
its CPU interpreter (TRITON_INTERPRET=1) on small kernels of this script that
call only tl.rand / tl.randint with the reference's argument shapes: an
integer seed argument plus the program id, and int32 column offsets. Nothing
of the reference is imported or run. The fixture pins oracle/sampler_oracle.py
(Philox4x32-10 and Triton's uint -> float conversion) against the dependency
itself.

Run: python tests/golden/make_sampler_golden.py   (CPU only, a few seconds)
"""
import os

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
COLS = 96          # offsets 0..COLS-1 plus a few large ones
ROWS = 4
BIG = [262143, 262144, 2 ** 20 + 7, 2 ** 31 - 1]
SEEDS = [0, 1234, 7919 * 13, 2 ** 31 - 3, 2 ** 40 + 5]


@triton.jit
def _rand_rows(Out, seed, Cols, n, NCOLS: tl.constexpr):
    row = tl.program_id(0)
    i = tl.arange(0, NCOLS)
    offs = tl.load(Cols + i, mask=i < n, other=0)
    u = tl.rand(seed + row, offs)
    tl.store(Out + row * NCOLS + i, u, mask=i < n)


@triton.jit
def _randint_rows(Out, seed, Cols, n, NCOLS: tl.constexpr):
    row = tl.program_id(0)
    i = tl.arange(0, NCOLS)
    offs = tl.load(Cols + i, mask=i < n, other=0)
    r = tl.randint(seed + row, offs)
    tl.store(Out + row * NCOLS + i, r, mask=i < n)


def main():
    cols = np.array(list(range(COLS)) + BIG, dtype=np.int32)
    n = cols.size
    ncols = triton.next_power_of_2(n)
    ct = torch.from_numpy(cols)
    rand = np.zeros((len(SEEDS), ROWS, n), dtype=np.float32)
    rint = np.zeros((len(SEEDS), ROWS, n), dtype=np.uint32)
    for si, seed in enumerate(SEEDS):
        out = torch.zeros(ROWS, ncols, dtype=torch.float32)
        _rand_rows[(ROWS,)](out, seed, ct, n, NCOLS=ncols)
        rand[si] = out[:, :n].numpy()
        outi = torch.zeros(ROWS, ncols, dtype=torch.int32)
        _randint_rows[(ROWS,)](outi, seed, ct, n, NCOLS=ncols)
        rint[si] = outi[:, :n].numpy().view(np.uint32)
    path = os.path.join(HERE, "sampler_rand.npz")
    np.savez_compressed(path, cols=cols, seeds=np.array(SEEDS, dtype=np.int64), rand=rand, randint=rint,
                        triton_version=np.array(triton.__version__))
    print(f"wrote {path}: seeds {SEEDS}, rows {ROWS}, {n} offsets")


if __name__ == "__main__":
    main()
