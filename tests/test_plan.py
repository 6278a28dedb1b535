"""Host-side launch plan (no device needed): the tile choice of the fitted
cost model, the two-launch tail split and the one-round 256 x 384 plan at a
column pitch, through gk_debug_plan.

The expected tiles are the measured best forced tiles of the 17-shape sweep the
model was fitted to (profiles/tile_choice.md), so a refit that loses one
of them fails here."""
import os

import pytest

import gemmkit_amd as gk

# (in, output kind, M, N, K bytes, batch) -> measured best tile
SWEEP = [
    (("i8", "i32", 4096, 4096, 4096, 1), "256x256w8m16"),
    (("i8", "q8", 2048, 11008, 4096, 1), "256x256w8m16"),
    (("i8", "i32", 2048, 11008, 4096, 1), "256x256w8m16"),
    (("i8", "i32", 8192, 8192, 1024, 1), "256x256w8m16"),
    (("i8", "i32", 1024, 1024, 8192, 1), "64x64"),
    (("i8", "i32", 3000, 5000, 2000, 1), "256x256w8m16"),
    (("i8", "q8", 4096, 4096, 4096, 1), "256x256w8m16"),
    (("bf16", "f32", 4096, 4096, 8192, 1), "256x256w8m16"),
    (("bf16", "f32", 512, 512, 256, 64), "256x256w8k128"),
    (("bf16", "bf16", 2048, 11008, 8192, 1), "256x256w8m16"),
    (("bf16", "bf16", 2048, 2048, 4096, 1), "128x128"),
    (("f32", "f32", 2048, 2048, 8192, 1), "128x128"),
    (("f32", "f32", 1024, 1024, 4096, 1), "64x64"),
    (("i8", "q8", 2048, 2816, 4096, 1), "128x128"),
    (("i8", "i32", 2048, 2816, 4096, 1), "256x128"),
    (("bf16", "bf16", 2048, 2816, 8192, 1), "256x128"),
    (("f32", "f32", 4096, 4096, 4096, 1), "256x256w8k128"),
]


@pytest.fixture
def clean_env(monkeypatch):
    monkeypatch.delenv("GEMMKIT_HIP_TILE", raising=False)
    monkeypatch.delenv("GEMMKIT_HIP_TAILSPLIT", raising=False)
    monkeypatch.delenv("GEMMKIT_HIP_WIDE", raising=False)
    monkeypatch.delenv("GEMMKIT_HIP_M16", raising=False)


@pytest.fixture
def no_wide(clean_env, monkeypatch):
    monkeypatch.setenv("GEMMKIT_HIP_WIDE", "0")


@pytest.fixture
def pick_only(no_wide, monkeypatch):
    monkeypatch.setenv("GEMMKIT_HIP_TAILSPLIT", "0")


@pytest.mark.parametrize("shape,best", SWEEP)
def test_model_picks_the_measured_best_tile(pick_only, shape, best):
    assert gk.debug_plan(*shape)[0] == best


def test_m16_tile_exclusions(pick_only, monkeypatch):
    # no f32 variant of the 16x16-MFMA tile
    assert gk.debug_plan("f32", "f32", 4096, 4096, 16384)[0] != "256x256w8m16"
    # bf16 contractions of at most 256 bytes stay on the 32x32 tiles (the
    # streaming kernel's summation order); int8 sums are exact either way
    assert gk.debug_plan("bf16", "f32", 4096, 4096, 256)[0] != "256x256w8m16"
    assert gk.debug_plan("bf16", "f32", 4096, 4096, 1024)[0] == "256x256w8m16"
    monkeypatch.setenv("GEMMKIT_HIP_M16", "0")
    assert gk.debug_plan("i8", "i32", 4096, 4096, 4096)[0] != "256x256w8m16"
    # ... and the one-round layer plan falls back to the 32x32 strip tile
    monkeypatch.delenv("GEMMKIT_HIP_WIDE", raising=False)
    monkeypatch.delenv("GEMMKIT_HIP_TAILSPLIT", raising=False)
    assert gk.debug_plan("i8", "q8", 2048, 11008, 4096)[0] == "256x352w8k128"


@pytest.mark.parametrize("shape,pitch,tile", [
    (("i8", "q8", 2048, 11008, 4096), 344, "256x352w8m16"),
    (("i8", "i32", 2048, 11008, 4096), 344, "256x352w8m16"),
    (("bf16", "bf16", 2048, 11008, 8192), 344, "256x384w8k128"),
    (("bf16", "f32", 2048, 11008, 8192), 344, "256x384w8k128"),
    (("i8", "i32", 4608, 4608, 4096), 336, "256x352w8m16"),
    (("i8", "q8", 2000, 11000, 4096), 344, "256x352w8m16"),
])
def test_wide_round_of_the_layer_shapes(clean_env, shape, pitch, tile):
    # 8 row tiles of 256 leave 32 tile columns per row for 256 CUs: 11008
    # columns at a 344-column pitch (4608: 18 row tiles, 14 columns at 336),
    # one launch of 256 x 352 strip tiles (int8) or 256 x 384 tiles (bf16:
    # the strip tile's main loop loses there)
    assert gk.debug_plan(*shape, pitches=True) == (tile, pitch, 0, tile, 0)


def test_wide_round_past_352_takes_the_384_tile(clean_env):
    # 2048 x 12000: 32 tile columns at a 376-column pitch
    assert gk.debug_plan("i8", "i32", 2048, 12000, 4096, pitches=True) == \
        ("256x384w8k128", 376, 0, "256x384w8k128", 0)


def test_no_wide_round_when_256_wide_tiles_fit_one_round(clean_env):
    # 4096^2: 16 x 16 tiles of 256 already make one round
    assert gk.debug_plan("i8", "i32", 4096, 4096, 4096, pitches=True) == \
        ("256x256w8m16", 0, 0, "256x256w8m16", 0)
    # batched products never take it (per element shape only), nor f32
    # inputs (2048 x 11008 x 4096: 1379 against 1328 us)
    assert gk.debug_plan("i8", "q8", 2048, 11008, 4096, 2)[0] != "256x384w8k128"
    assert gk.debug_plan("f32", "f32", 2048, 11008, 16384)[0] != "256x384w8k128"


@pytest.mark.parametrize("shape,plan", [
    (("i8", "q8", 2048, 11008, 4096), ("256x256w8m16", 8192, "128x96k128o2")),
    (("i8", "i32", 2048, 11008, 4096), ("256x256w8m16", 8192, "128x192k128")),
    # bf16 splits keep the 32x32 tiles' summation order throughout
    (("bf16", "bf16", 2048, 11008, 8192), ("256x256w8k128", 8192, "128x192k128")),
])
def test_tail_split_of_the_layer_shapes(no_wide, shape, plan):
    # 8 x 43 tiles of 256: the first 32 tile columns fill one round of 256
    # CUs; the rest (2048 x 2816) runs as one round of 16 x 16 tiles of
    # 128 x 192 at a 176-column pitch (measured against the 128-wide rests:
    # i32 98.4 against 101.5 us, bf16 156.6 against 170.7), or, requantized,
    # 16 x 32 tiles of 128 x 96 at an 88-column pitch, two per CU (103.2
    # against 106.8 with the 128 x 192 rest)
    assert gk.debug_plan(*shape) == plan


def test_no_split_for_one_round(clean_env):
    assert gk.debug_plan("i8", "i32", 4096, 4096, 4096)[1] == 0
    assert gk.debug_plan("bf16", "f32", 4096, 4096, 8192)[1] == 0


def test_split_switches(no_wide, monkeypatch):
    monkeypatch.setenv("GEMMKIT_HIP_TAILSPLIT", "0")
    assert gk.debug_plan("i8", "q8", 2048, 11008, 4096)[1] == 0
    monkeypatch.delenv("GEMMKIT_HIP_TAILSPLIT")
    monkeypatch.setenv("GEMMKIT_HIP_TILE", "256x256")
    assert gk.debug_plan("i8", "q8", 2048, 11008, 4096) == ("256x256", 0, "256x256")
    # batched products never split (the split is per element shape only)
    monkeypatch.delenv("GEMMKIT_HIP_TILE")
    assert gk.debug_plan("i8", "q8", 2048, 11008, 4096, 2)[1] == 0


def test_forced_wide_tile_takes_the_round_pitch(clean_env, monkeypatch):
    monkeypatch.setenv("GEMMKIT_HIP_TILE", "256x384w8k128")
    assert gk.debug_plan("i8", "i32", 2048, 11008, 4096, pitches=True) == \
        ("256x384w8k128", 344, 0, "256x384w8k128", 0)
    monkeypatch.setenv("GEMMKIT_HIP_TILE", "256x352w8k128")
    assert gk.debug_plan("i8", "i32", 2048, 11008, 4096, pitches=True) == \
        ("256x352w8k128", 344, 0, "256x352w8k128", 0)
    monkeypatch.setenv("GEMMKIT_HIP_TILE", "256x352w8m16")
    assert gk.debug_plan("i8", "i32", 2048, 11008, 4096, pitches=True) == \
        ("256x352w8m16", 344, 0, "256x352w8m16", 0)
    # no pitch in [192, 384] makes one round: plain 384-wide tiles
    assert gk.debug_plan("i8", "i32", 300, 500, 4096, pitches=True)[1] == 0


def test_bad_arguments():
    with pytest.raises(gk.GemmkitError):
        gk.debug_plan("i8", "i32", 0, 16, 16)


# bf16: the 16x16-MFMA tile sums in another order than the 32x32 tiles, so a
# batch must take the tile family its element's standalone plan takes, or a
# batched element would differ from its standalone call in the last bits
# (src/api/batched.rs:172-176).  Every shape x K x batch of this grid.
@pytest.mark.parametrize("kind", ["f32", "bf16"])
def test_bf16_batch_takes_the_standalone_tile_family(clean_env, kind):
    sides = [256, 512, 768, 1024, 1536, 2048, 3072, 4096]
    bad = []
    for m in sides:
        for n in sides:
            for kbytes in (512, 1024, 4096, 8192):
                one = gk.debug_plan("bf16", kind, m, n, kbytes, 1)[0] == "256x256w8m16"
                for batch in (2, 4, 8, 16, 64):
                    many = gk.debug_plan("bf16", kind, m, n, kbytes, batch)[0] == "256x256w8m16"
                    if many != one:
                        bad.append((m, n, kbytes, batch, one, many))
    assert not bad, bad[:5]


def test_wide_tiles_keep_their_rows_within_32bit_offsets(clean_env):
    # 8192 x 2640 int8 products take the one-round strip tile (pitch 336) with
    # packed rows; with B^T rows 8 MB apart its 352 rows would span 2.8 GB of
    # 32-bit buffer offsets, so the plan must not take the wide tiles then.
    assert gk.debug_plan("i8", "i32", 8192, 2640, 4112, pitches=True)[0] == "256x352w8m16"
    for ld in (8000016, 6 << 20):
        t = gk.debug_plan("i8", "i32", 8192, 2640, 4112, ld_b=ld)[0]
        assert t not in ("256x352w8k128", "256x384w8k128", "256x352w8m16"), (ld, t)
    # the largest stride that still fits keeps it
    ld_max = (0x7FFFFFF0 - 4112) // 351
    assert gk.debug_plan("i8", "i32", 8192, 2640, 4112, ld_b=ld_max)[0] == "256x352w8m16"
