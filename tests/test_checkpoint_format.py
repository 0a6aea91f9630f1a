"""The checkpoint format on the host: manifest JSON, validation, naming and path rules.

Mirrors the reference's format tests (``tests/unit/test_checkpoint_format.py``): a
manifest round-trips through JSON unchanged, is refused when incomplete, of an
unknown version, overlapping, gapped or pointing at a file without an integrity
record; file names follow ``rank-NNNNN.pt`` and paths stay inside the directory.
Files are written with CPU tensors here; the device load path is a GPU test.
"""

from __future__ import annotations

import hashlib
import json
import os

import pytest
import torch

from hybrid_training_amd import (
    CheckpointError,
    CheckpointManifest,
    CheckpointVersionError,
    FileRecord,
    IncompleteCheckpointError,
    ShardFileCache,
    ShardRecord,
    ShardRange,
    TensorRecord,
    checkpoint_directory_name,
    describe_reshard,
    verify_files,
    write_checkpoint,
)
from hybrid_training_amd.errors import CheckpointCorruptionError
from hybrid_training_amd.manifest import (
    MANIFEST_FILENAME,
    file_digest,
    resolve_inside,
    staging_directory_name,
    step_from_directory_name,
)


def _manifest(complete=True):
    m = CheckpointManifest(step=7, writer_world_size=2, complete=complete)
    rec = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32")
    m.add_shard(rec, ShardRecord(rank=0, file="rank-00000.pt", offset=0, length=6, key="model::w@0"))
    m.add_shard(rec, ShardRecord(rank=1, file="rank-00001.pt", offset=6, length=6, key="model::w@6"))
    m.files["rank-00000.pt"] = FileRecord("rank-00000.pt", "0" * 64, 10)
    m.files["rank-00001.pt"] = FileRecord("rank-00001.pt", "1" * 64, 10)
    return m


def test_manifest_round_trip_and_validation():
    m = _manifest()
    m.validate()
    again = CheckpointManifest.from_dict(json.loads(m.to_json()))
    assert again.as_dict() == m.as_dict()
    assert again.tensors["w"].shards_overlapping(
        __import__("hybrid_training_amd").ShardRange(4, 4))[0][1].length == 2
    with pytest.raises(IncompleteCheckpointError, match="not marked complete"):
        _manifest(complete=False).validate()
    bad = _manifest()
    bad.format_version = "9.9"
    with pytest.raises(CheckpointVersionError):
        bad.validate()
    missing = _manifest()
    del missing.files["rank-00001.pt"]
    with pytest.raises(IncompleteCheckpointError, match="no integrity record"):
        missing.validate()
    with pytest.raises(CheckpointCorruptionError, match="differently"):
        _manifest().add_shard(TensorRecord(key="w", name="w", global_shape=(4, 4), dtype="torch.float32"),
                              ShardRecord(rank=2, file="rank-00002.pt", offset=0, length=1, key="x"))
    with pytest.raises(CheckpointError, match="malformed"):
        CheckpointManifest.from_dict({"tensors": {}})


def test_names_and_paths(tmp_path):
    assert checkpoint_directory_name(100) == "checkpoint-step-000100"
    assert step_from_directory_name("checkpoint-step-000100") == 100
    assert step_from_directory_name("checkpoint-step-1") is None
    assert staging_directory_name("checkpoint-step-000001", "ab").startswith(".staging-")
    assert resolve_inside(tmp_path, "rank-00000.pt") == (tmp_path / "rank-00000.pt").resolve()
    with pytest.raises(CheckpointError, match="escapes"):
        resolve_inside(tmp_path, "../outside.pt")
    os.symlink("/etc", tmp_path / "link")
    with pytest.raises(CheckpointError, match="escapes"):
        resolve_inside(tmp_path, "link/passwd")
    (tmp_path / "abc").write_bytes(b"abc")
    assert file_digest(tmp_path / "abc") == hashlib.sha256(b"abc").hexdigest()
    with pytest.raises(IncompleteCheckpointError, match="no manifest found"):
        CheckpointManifest.read(tmp_path / MANIFEST_FILENAME)


def _cpu_checkpoint(tmp_path):
    """Two writers of a (3, 4) tensor, written with CPU tensors."""
    data = torch.arange(12, dtype=torch.float32)
    shards = []
    for rank in (0, 1):
        piece = data[6 * rank : 6 * rank + 6].clone()
        records = [{"key": "w", "name": "w", "global_shape": [3, 4], "dtype": "torch.float32",
                    "category": "model", "partition_dim": None, "tensor_parallel_size": 1,
                    "tensor_parallel_rank": 0, "state_name": "", "rank": rank, "file": f"rank-0000{rank}.pt",
                    "offset": 6 * rank, "length": 6, "storage_key": f"model::w@{6 * rank}"}]
        shards.append((rank, {f"model::w@{6 * rank}": piece}, records, {"step": 3}))
    return write_checkpoint(tmp_path, 3, shards), data


def test_written_checkpoint_is_complete_and_verified(tmp_path):
    path, data = _cpu_checkpoint(tmp_path)
    assert path.name == "checkpoint-step-000003" and not any(p.name.startswith(".staging") for p in tmp_path.iterdir())
    manifest = CheckpointManifest.read(path / MANIFEST_FILENAME)
    manifest.validate()
    meta = json.loads((path / "metadata.json").read_text())
    assert meta["optimizer_scalars"] == {"step": 3} and manifest.step == 3
    cache = ShardFileCache(path, manifest, device="cpu")
    assert torch.equal(cache.get("rank-00001.pt")["model::w@6"], data[6:])
    assert cache.loaded_files == ("rank-00001.pt",)
    with pytest.raises(CheckpointError, match="already exists"):
        _cpu_checkpoint(tmp_path)


def test_failed_publish_renames_nothing_and_keeps_the_staging_directory(tmp_path):
    """``checkpoint/writer.py:290-307``: when the manifest cannot be validated (here two
    writers claim the same elements) nothing is renamed into place, the error is the
    reference's, and the staging directory stays for inspection."""
    data = torch.arange(12, dtype=torch.float32)
    shards = []
    for rank in (0, 1):
        records = [{"key": "w", "name": "w", "global_shape": [3, 4], "dtype": "torch.float32",
                    "category": "model", "partition_dim": None, "tensor_parallel_size": 1,
                    "tensor_parallel_rank": 0, "state_name": "", "rank": rank, "file": f"rank-0000{rank}.pt",
                    "offset": 0, "length": 12, "storage_key": "model::w@0"}]
        shards.append((rank, {"model::w@0": data.clone()}, records, {"step": 1}))
    with pytest.raises(CheckpointError, match="publishing the checkpoint failed") as info:
        write_checkpoint(tmp_path, 1, shards)
    assert "overlap" in str(info.value)
    assert not (tmp_path / "checkpoint-step-000001").exists()
    staged = [p for p in tmp_path.iterdir() if p.name.startswith(".staging")]
    assert len(staged) == 1 and staged[0].name in str(info.value)


def test_corruption_is_detected(tmp_path):
    path, _ = _cpu_checkpoint(tmp_path)
    manifest = CheckpointManifest.read(path / MANIFEST_FILENAME)
    target = path / "rank-00000.pt"
    raw = bytearray(target.read_bytes())
    raw[len(raw) // 2] ^= 0xFF
    target.write_bytes(bytes(raw))
    with pytest.raises(CheckpointCorruptionError, match="checksum"):
        ShardFileCache(path, manifest, device="cpu").get("rank-00000.pt")
    target.write_bytes(bytes(raw[:-7]))
    with pytest.raises(CheckpointCorruptionError, match="wrong size"):
        ShardFileCache(path, manifest, device="cpu").get("rank-00000.pt")
    target.unlink()
    with pytest.raises(IncompleteCheckpointError, match="missing"):
        ShardFileCache(path, manifest, device="cpu").get("rank-00000.pt")
    with pytest.raises(CheckpointError, match="naming rule"):
        ShardFileCache(path, manifest, device="cpu").get("../rank-00000.pt")


def test_verify_files_and_describe_reshard(tmp_path):
    """``verify_files`` digests every referenced file and refuses a corrupt or missing one;
    ``describe_reshard`` lists the saved shards a read touches (``reshard.py:308-421``)."""
    path, _ = _cpu_checkpoint(tmp_path)
    manifest = CheckpointManifest.read(path / MANIFEST_FILENAME)
    digests = verify_files(path, manifest)
    assert set(digests) == {"rank-00000.pt", "rank-00001.pt"}
    assert all(d == file_digest(path / f) for f, d in digests.items())
    assert set(verify_files(path, manifest, filenames={"rank-00001.pt"})) == {"rank-00001.pt"}
    plan = describe_reshard(manifest, "w", ShardRange(4, 4))
    assert plan["global_shape"] == [3, 4] and plan["wanted"] == [4, 4]
    assert [(s["saved_rank"], s["overlap"]) for s in plan["sources"]] == [(0, [4, 2]), (1, [6, 2])]
    with pytest.raises(CheckpointError, match="unknown tensor key"):
        describe_reshard(manifest, "nope", ShardRange(0, 1))
    target = path / "rank-00001.pt"
    data = bytearray(target.read_bytes())
    data[-1] ^= 0xFF
    target.write_bytes(bytes(data))
    with pytest.raises(CheckpointCorruptionError, match="checksum"):
        verify_files(path, manifest)
    target.unlink()
    with pytest.raises(IncompleteCheckpointError, match="missing"):
        verify_files(path, manifest)
