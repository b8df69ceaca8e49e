"""DSQG offset tables.

* ``OFFSETS_V3`` -- kernels/dsqg_attention_v3.py:47-49 (``ALL_OFFSETS``): the dense window
  0..32 plus eleven semi-dyadic long-range taps, 44 offsets.  The same table is built in
  train/train_2048_condU.py:98-102 and kernels/dsqg_attention_v2.py:40-42.
* ``OFFSETS_J46`` -- V3 plus {2048, 3072} (46 offsets), for N = 4096.
* ``OFFSETS_J47`` -- train/train_4096_13m_condU.py:88-93: V3 plus {2048, 3072, 4096}.

The kernels take the table as data (``offsets`` argument); these are the named defaults.
"""

SPARSE_V3 = (48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536)
OFFSETS_V3 = tuple(range(33)) + SPARSE_V3
OFFSETS_J46 = OFFSETS_V3 + (2048, 3072)
OFFSETS_J47 = OFFSETS_V3 + (2048, 3072, 4096)
ALL_OFFSETS = list(OFFSETS_V3)  # name used by the reference module

assert len(OFFSETS_V3) == 44 and len(OFFSETS_J46) == 46 and len(OFFSETS_J47) == 47

_BY_COUNT = {44: OFFSETS_V3, 46: OFFSETS_J46, 47: OFFSETS_J47}


def default_offsets(J: int) -> tuple:
    """The named table with J entries (44, 46 or 47)."""
    if J not in _BY_COUNT:
        raise AssertionError(
            f"no default offset table has {J} entries (44, 46, 47); pass offsets= explicitly")
    return _BY_COUNT[J]


def validate(offsets) -> tuple:
    """Return the table as a tuple of ints; it must be strictly increasing from 0."""
    offs = tuple(int(o) for o in offsets)
    if not offs or offs[0] != 0 or any(b <= a for a, b in zip(offs, offs[1:])):
        raise AssertionError(f"offsets must be strictly increasing and start at 0: {offs}")
    return offs


def long_range_taps(offsets) -> int:
    """Taps beyond the dense window: the table's leading run 0, 1, ..., W (W <= 32) is the
    window the kernels stage whole; the rest (NS = J - W - 1) are gathered row blocks, whose
    softmax weights the bf16 forward saves for the backward ([B,H,NS,N])."""
    offs = tuple(int(o) for o in offsets)
    W = 0
    while W + 1 < len(offs) and W + 1 <= 32 and offs[W + 1] == W + 1:
        W += 1
    return len(offs) - W - 1
