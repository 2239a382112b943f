"""Checkpoint reader checks on the host (no device), against the reference's hostile corpus and its format rules.

The target is the reference's CheckpointHostileTests model, a Linear(2, 2) with bias: state weight [2,2] then
bias [2] (CheckpointHostileTests.cs:13-16). Each of the reference's 42 hostile files must fail with the kind in
its name (CheckpointHostileTests.cs:60-115); the valid base file, assembled here from the documented layout, must
pass; every single-byte corruption of it must pass or fail with a checkpoint kind, never another error
(CheckpointTests.cs:170-183).
"""
import glob
import os
import struct

import pytest

from conftest import GOLDEN
from gpu_util import load_pkg

TARGET = [("weight", "f32", [2, 2]), ("bias", "f32", [2])]
BASE = ('{"format":"onemodel-checkpoint","version":1,"model":[{"name":"weight","dtype":"f32","shape":[2,2],'
        '"offset":0,"length":16},{"name":"bias","dtype":"f32","shape":[2],"offset":64,"length":8}],"extra":[]}')


def assemble(manifest: bytes, data: bytes) -> bytes:
    """The documented frame: 64-byte header, manifest, zero padding to a multiple of 64, data region."""
    data_offset = (64 + len(manifest) + 63) // 64 * 64
    head = b"ONEMCKPT" + struct.pack("<IIQQQQQQ", 1, 0, 64, len(manifest), data_offset, len(data),
                                     data_offset + len(data), 0)
    return head + manifest + bytes(data_offset - 64 - len(manifest)) + data


def base_data() -> bytes:
    return struct.pack("<4f", 1, 2, 3, 4) + bytes(48) + struct.pack("<2f", 5, 6)


def check(pkg, tmp_path, blob: bytes, name="x.ckpt"):
    p = tmp_path / name
    p.write_bytes(blob)
    pkg.checkpoint_check(str(p), TARGET)


@pytest.fixture(scope="module")
def pkg():
    return load_pkg()


HOSTILE = sorted(glob.glob(os.path.join(GOLDEN, "checkpoint_hostile", "*.ckpt")))


def test_hostile_corpus_is_complete():
    assert len(HOSTILE) == 42


@pytest.mark.parametrize("path", HOSTILE, ids=lambda p: os.path.basename(p)[:-5])
def test_hostile_file_fails_with_its_kind(pkg, path):
    kind = os.path.basename(path).split("-")[0]
    with pytest.raises(pkg.CheckpointError) as e:
        pkg.checkpoint_check(path, TARGET)
    assert e.value.kind == kind, str(e.value)


def test_base_case_loads(pkg, tmp_path):
    check(pkg, tmp_path, assemble(BASE.encode(), base_data()))


def test_extra_optimizer_fields_and_whitespace_are_accepted(pkg, tmp_path):
    m = BASE.replace('"extra":[]', '"extra":[{"key":"step","value":6}],"optimizer":{"kind":"adam"}')
    check(pkg, tmp_path, assemble((" \n" + m + "\t").encode(), base_data()))


def test_every_single_byte_corruption_is_typed(pkg, tmp_path):
    good = assemble(BASE.encode(), base_data())
    p = tmp_path / "c.ckpt"
    for i in range(len(good)):
        bad = bytearray(good)
        bad[i] ^= 0xFF
        p.write_bytes(bytes(bad))
        try:
            pkg.checkpoint_check(str(p), TARGET)
        except pkg.CheckpointError:
            pass


def test_header_lies(pkg, tmp_path):
    good = bytearray(assemble(BASE.encode(), base_data()))
    for at, value in ((24, 2 ** 64 - 1), (32, 65), (48, len(good) + 1), (40, 0)):
        bad = bytearray(good)
        bad[at:at + 8] = struct.pack("<Q", value)
        with pytest.raises(pkg.CheckpointError) as e:
            check(pkg, tmp_path, bytes(bad))
        assert e.value.kind == "BadHeader"


@pytest.mark.parametrize("manifest,kind", [
    ('{"format":"onemodel-checkpoint","version":1,"model":[],"extra":[]}', "Mismatch"),
    (BASE.replace('"length":16', '"length":16.0'), "BadManifest"),
    (BASE.replace('"length":16', '"length":1e1'), "BadManifest"),
    (BASE.replace('"weight"', '"we\\ud800ight"'), "BadManifest"),
    (BASE.replace('"weight"', '"we\\u0069ght"'), None),  # an escaped 'i' is the same name
    (BASE + ",", "BadManifest"),
    (BASE.replace('"extra":[]', '"extra":[{"key":"k","value":"v"}]'), "BadManifest"),
    (BASE.replace('"shape":[2,2]', '"shape":[2,2147483648]'), "BadManifest"),
    (BASE.replace('"shape":[2]', '"shape":[2,1]'), "Mismatch"),
    (BASE.replace('"offset":64', '"offset":8'), None),  # any in-bounds offset is accepted
])
def test_manifest_rules(pkg, tmp_path, manifest, kind):
    blob = assemble(manifest.encode(), base_data())
    if kind is None:
        check(pkg, tmp_path, blob)
    else:
        with pytest.raises(pkg.CheckpointError) as e:
            check(pkg, tmp_path, blob)
        assert e.value.kind == kind, str(e.value)


def test_non_seekable_input_is_refused(pkg):
    with pytest.raises(pkg.CheckpointError) as e:
        pkg.checkpoint_check("/dev/null", TARGET)
    assert e.value.kind == "UnsupportedStream"


def test_missing_file_is_not_a_checkpoint_kind(pkg, tmp_path):
    with pytest.raises(pkg.OmError) as e:
        pkg.checkpoint_check(str(tmp_path / "absent.ckpt"), TARGET)
    assert not isinstance(e.value, pkg.CheckpointError)
