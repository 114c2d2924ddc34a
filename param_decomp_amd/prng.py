"""JAX-compatible threefry2x32 key derivation on the host (scalar integer work).

Mirrors `jax.random.PRNGKey` / `split` / `fold_in` as the reference uses them
(`param_decomp/param_decomp/core/run.py:978-979, 1141`, `core/train.py:434-486`,
`core/masking.py:148-167`). Keys are `(k0, k1)` uint32 pairs. Array draws from a key run
on the GPU (`masking.uniform_like`).

- `PRNGKey(seed)` = `(0, seed)` for a 32-bit seed.
- `fold_in(key, d)` = threefry2x32(key, (0, d)).
- `split(key, n)`: in the partitionable layout (JAX >= 0.5 default) subkey i is
  threefry2x32(key, (hi(i), lo(i))); in the original layout the 2n counter words
  iota(2n) are halved into the block's two inputs and the outputs concatenated.
"""

from __future__ import annotations

Key = tuple[int, int]
_M = 0xFFFFFFFF
_R = (13, 15, 26, 6, 17, 29, 16, 24)

PARTITIONABLE = True


def _rotl(x: int, r: int) -> int:
    return ((x << r) | (x >> (32 - r))) & _M


def threefry2x32(key: Key, x0: int, x1: int) -> Key:
    k0, k1 = key[0] & _M, key[1] & _M
    ks = (k0, k1, k0 ^ k1 ^ 0x1BD11BDA)
    x0 = (x0 + ks[0]) & _M
    x1 = (x1 + ks[1]) & _M
    for b in range(5):
        for i in range(4):
            x0 = (x0 + x1) & _M
            x1 = _rotl(x1, _R[(b & 1) * 4 + i]) ^ x0
        x0 = (x0 + ks[(b + 1) % 3]) & _M
        x1 = (x1 + ks[(b + 2) % 3] + b + 1) & _M
    return (x0, x1)


def PRNGKey(seed: int) -> Key:
    if not 0 <= seed <= _M:
        raise ValueError("seed must be a non-negative 32-bit integer")
    return (0, seed)


def fold_in(key: Key, data: int) -> Key:
    return threefry2x32(key, 0, data & _M)


def split(key: Key, num: int = 2, *, partitionable: bool | None = None) -> list[Key]:
    part = PARTITIONABLE if partitionable is None else partitionable
    if part:
        return [threefry2x32(key, (i >> 32) & _M, i & _M) for i in range(num)]
    half = num  # iota(2*num) halves: (c[i], c[num+i]) feed block i
    outs = [threefry2x32(key, i, half + i) for i in range(num)]
    flat = [o[0] for o in outs] + [o[1] for o in outs]
    return [(flat[2 * i], flat[2 * i + 1]) for i in range(num)]
