"""Threefry-2x32 and JAX's key/bits/uniform layout, restated in NumPy (oracle only).

The reference draws every stochastic mask with `jax.random.uniform`
(`param_decomp/param_decomp/core/linear_plan.py:80-106`, called from
`core/masking.py:135-140`) under JAX's default `threefry2x32` PRNG, and derives keys
with `PRNGKey` / `split` / `fold_in` (`core/run.py:978-979, 1141`;
`core/train.py:434-486`; `core/masking.py:148-171`).

JAX is a third-party dependency (jax 0.11.1, `param_decomp/pyproject.toml:17`) that is
not importable here. Its published algorithm, restated:

- Block function: Threefry-2x32 with 20 rounds (Salmon, Moraes, Dror, Shaw, "Parallel
  random numbers: as easy as 1, 2, 3", SC'11), rotation constants
  (13,15,26,6,17,29,16,24), key-schedule parity constant 0x1BD11BDA.
- `PRNGKey(seed)` for a 32-bit seed is `(0, seed)`.
- `fold_in(key, d)` is `block(key, (0, d))`.
- Two counter layouts ("original" and "partitionable"; JAX >= 0.5 defaults to
  partitionable):
  * partitionable: element i (row-major flat index, a 64-bit counter split into
    hi/lo words) gets `block(key, (hi(i), lo(i)))`; `split(key, n)[i]` is that block
    output, which makes it equal to `fold_in(key, i)`; 32-bit random bits are
    `x0 ^ x1`, 8/16-bit bits are the low byte/half of `x0 ^ x1`.
  * original: `threefry_2x32(key, iota(2n))` splits the counter vector into two
    halves, feeds (c[i], c[n+i]) to the block and concatenates the two output words;
    `split` draws from `iota(2n)` reshaped to `[n, 2]`; 8/16-bit bits are successive
    little-endian sub-words of the 32-bit stream.
- `uniform(key, shape, dtype)`: draw `nbits` random bits (8 when the mantissa has fewer
  than 8 bits, as for bfloat16), shift right by `nbits_drawn - nmant`, OR in the bit
  pattern of 1.0, bitcast and subtract 1.0. fp32: `(b >> 9) * 2^-23`; bf16:
  `((b & 0xff) >> 1) * 2^-7`.
"""

from __future__ import annotations

import numpy as np

ROTATIONS = (13, 15, 26, 6, 17, 29, 16, 24)
PARITY = np.uint32(0x1BD11BDA)
M32 = 0xFFFFFFFF


def _rotl(x: np.ndarray, r: int) -> np.ndarray:
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def threefry2x32(key: tuple[int, int], x0, x1) -> tuple[np.ndarray, np.ndarray]:
    """Threefry-2x32-20 block function, vectorized over counter words (x0, x1)."""
    k0 = np.uint32(key[0] & M32)
    k1 = np.uint32(key[1] & M32)
    ks = (k0, k1, np.uint32(k0 ^ k1 ^ PARITY))
    x0 = np.asarray(x0, dtype=np.uint32).copy()
    x1 = np.asarray(x1, dtype=np.uint32).copy()
    with np.errstate(over="ignore"):
        x0 = x0 + ks[0]
        x1 = x1 + ks[1]
        for block in range(5):
            rots = ROTATIONS[:4] if block % 2 == 0 else ROTATIONS[4:]
            for r in rots:
                x0 = x0 + x1
                x1 = _rotl(x1, r)
                x1 = x1 ^ x0
            x0 = x0 + ks[(block + 1) % 3]
            x1 = x1 + ks[(block + 2) % 3] + np.uint32(block + 1)
    return x0, x1


def prng_key(seed: int) -> tuple[int, int]:
    """`jax.random.PRNGKey(seed)` for a non-negative 32-bit seed: `(0, seed)`."""
    assert 0 <= seed <= M32
    return (0, seed)


def fold_in(key: tuple[int, int], data: int) -> tuple[int, int]:
    """`jax.random.fold_in(key, data)` = `block(key, (0, uint32(data)))`."""
    y0, y1 = threefry2x32(key, np.uint32(0), np.uint32(data & M32))
    return (int(y0), int(y1))


def split(key: tuple[int, int], n: int = 2, *, partitionable: bool = True) -> list[tuple[int, int]]:
    """`jax.random.split(key, n)` in either counter layout."""
    if partitionable:
        idx = np.arange(n, dtype=np.uint64)
        y0, y1 = threefry2x32(key, (idx >> np.uint64(32)).astype(np.uint32), idx.astype(np.uint32))
        return [(int(a), int(b)) for a, b in zip(y0, y1)]
    out = _threefry_2x32_vector(key, np.arange(2 * n, dtype=np.uint32))
    out = out.reshape(n, 2)
    return [(int(a), int(b)) for a, b in out]


def _threefry_2x32_vector(key: tuple[int, int], count: np.ndarray) -> np.ndarray:
    """JAX's `threefry_2x32(keypair, count)`: halves of the (even-padded) counter vector
    form the two block words; the two output words are concatenated."""
    count = np.asarray(count, dtype=np.uint32).ravel()
    odd = count.size % 2
    if odd:
        count = np.concatenate([count, np.zeros(1, np.uint32)])
    half = count.size // 2
    y0, y1 = threefry2x32(key, count[:half], count[half:])
    out = np.concatenate([y0, y1])
    return out[:-1] if odd else out


def random_bits(key: tuple[int, int], bit_width: int, shape, *, partitionable: bool = True) -> np.ndarray:
    """`jax.random.bits`-style raw bits (uint8/16/32) of `shape`."""
    shape = tuple(int(s) for s in shape)
    size = int(np.prod(shape, dtype=np.int64)) if shape else 1
    dtype = {8: np.uint8, 16: np.uint16, 32: np.uint32}[bit_width]
    if partitionable:
        idx = np.arange(size, dtype=np.uint64)
        y0, y1 = threefry2x32(key, (idx >> np.uint64(32)).astype(np.uint32), idx.astype(np.uint32))
        bits = y0 ^ y1
        return bits.astype(dtype).reshape(shape)
    max_count = -(-bit_width * size // 32)
    assert max_count < M32, "oracle handles the single-block original layout only"
    words = _threefry_2x32_vector(key, np.arange(max_count, dtype=np.uint32))
    if bit_width == 32:
        return words.reshape(shape)
    per = 32 // bit_width
    mask = (1 << bit_width) - 1
    sub = np.stack([(words >> np.uint32(bit_width * i)) & np.uint32(mask) for i in range(per)], axis=1)
    return sub.reshape(-1)[:size].astype(dtype).reshape(shape)


def uniform_bits_to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    """JAX `_uniform`'s mantissa trick, returned as float64 values (exact)."""
    if dtype == "float32":
        mant = (bits.astype(np.uint32) >> np.uint32(9)).astype(np.float64)
        return mant * 2.0**-23
    if dtype == "bfloat16":
        mant = ((bits.astype(np.uint32) & np.uint32(0xFF)) >> np.uint32(1)).astype(np.float64)
        return mant * 2.0**-7
    raise ValueError(dtype)


def uniform(key: tuple[int, int], shape, dtype: str = "float32", *, partitionable: bool = True) -> np.ndarray:
    """`jax.random.uniform(key, shape, dtype)` on [0, 1), as exact float64 values.

    The fp32 partitionable draw equals the reference's stored JAX draws
    (`tests/targets/stacked_parity/stacked_fixtures.npz`, `src::*`) bit for bit; the
    bf16 draw is parity unpinned against JAX (no stored bf16 draw exists)."""
    nbits = {"float32": 32, "bfloat16": 8}[dtype]
    return uniform_bits_to_float(random_bits(key, nbits, shape, partitionable=partitionable), dtype)


def randint(key: tuple[int, int], shape, minval: int, maxval: int, *, partitionable: bool = True) -> np.ndarray:
    """`jax.random.randint(key, shape, minval, maxval)` for int32 (JAX's `_randint`):
    `k1, k2 = split(key)`; 32 high and 32 low random bits from `k1` and `k2`; with
    `span = maxval - minval` (1 when maxval <= minval) the offset is
    `((hi % span) * m + lo % span) % span`, `m = (2^16 % span)^2 % span`, i.e. the
    64-bit value `hi * 2^32 + lo` reduced mod span in 32-bit arithmetic.

    The key/bit assignment follows the published JAX source; no golden vector exists
    for it here (parity unpinned beyond the modular identity and range checks)."""
    k1, k2 = split(key, partitionable=partitionable)
    hi = random_bits(k1, 32, shape, partitionable=partitionable).astype(np.uint64)
    lo = random_bits(k2, 32, shape, partitionable=partitionable).astype(np.uint64)
    span = np.uint64(maxval - minval if maxval > minval else 1)
    mult = (np.uint64(65536) % span) * (np.uint64(65536) % span) % span
    off = ((hi % span) * mult + lo % span) % span
    return (np.int64(minval) + off.astype(np.int64)).astype(np.int32)
