"""Checkpoint format and resume logic on the CPU: the oracle restatement against the reference's
own checkpoint tests, the library's FindLatest against the oracle, and AdamW's decay rule on the
reference's parameter names (which fixes which engine tensors are weight-decayed)."""
import os

import numpy as np
import pytest

from oracle import checkpoint as ock
from sharpmind_amd.engine import find_latest_checkpoint
from sharpmind_amd.model import ModelConfig


def test_oracle_roundtrip_duplicate_names_in_order(tmp_path):
    """CheckpointTests.RoundTrip_RestoresDuplicateNamedParametersInOrder (CheckpointTests.cs:15-48)."""
    a = np.array([1, 2, 3], np.float32)
    b = np.array([4, 5], np.float32)
    e = np.array([9], np.float32)
    ock.save(str(tmp_path), [("norm.weight", a), ("norm.weight", b), ("embed", e)])
    qa, qb, qe = np.zeros(3, np.float32), np.zeros(2, np.float32), np.zeros(1, np.float32)
    ock.load(str(tmp_path), [("norm.weight", qa), ("norm.weight", qb), ("embed", qe)])
    assert qa.tolist() == [1, 2, 3] and qb.tolist() == [4, 5] and qe.tolist() == [9]


def test_oracle_shape_mismatch_names_tensor(tmp_path):
    """CheckpointTests.Load_Throws_OnTensorShapeMismatch (CheckpointTests.cs:90-107)."""
    ock.save(str(tmp_path), [("layer.weight", np.zeros(4, np.float32))])
    with pytest.raises(ock.ShapeMismatch) as ei:
        ock.load(str(tmp_path), [("layer.weight", np.zeros(3, np.float32))])
    msg = str(ei.value)
    assert "layer.weight" in msg and "4" in msg and "3" in msg


def test_oracle_skips_unknown_and_reads_meta(tmp_path):
    ock.save(str(tmp_path), [("position_embedding", np.ones(5, np.float32)), ("w", np.full(2, 7, np.float32))],
             optimizer=(3, 0.5, [np.ones(2, np.float32)], [np.full(2, 2, np.float32)]), step=11, loss=1.25,
             note="final")
    w = np.zeros(2, np.float32)
    opt = {}
    step, loss, note = ock.load(str(tmp_path), [("w", w)], optimizer=opt)
    assert w.tolist() == [7, 7] and (step, loss, note) == (11, 1.25, "final")
    # LoadState skips the stored AdamW step: meta.json's step is authoritative (AdamW.cs:107-110)
    assert opt["step"] == 11 and opt["lr"] == 0.5 and opt["m"][0].tolist() == [1, 1]


def test_oracle_read_meta_defaults(tmp_path):
    """ReadMeta without meta.json: step 0, loss NaN (Checkpoint.cs:95-96)."""
    step, loss, note = ock.read_meta(str(tmp_path))
    assert step == 0 and np.isnan(loss) and note is None


FIND_LATEST_CASES = [
    # CheckpointTests.FindLatest_PicksHighestStepDirectory (CheckpointTests.cs:51-70)
    (["step-0000002", "step-0000001", "step-0000009", "step-0000009-final", "step-0000123", "unrelated"],
     "step-0000123"),
    (["step-0000009", "step-0000009-final"], "step-0000009-final"),
    # unpadded names: the reference's ParseStep returns 0 for every "step-" name, so the
    # ordinal-greatest name wins ("step-9" over "step-10")
    (["step-10", "step-9"], "step-9"),
    (["unrelated", "other"], None),
    ([], None),
]


@pytest.mark.parametrize("names,want", FIND_LATEST_CASES)
def test_find_latest_library_matches_oracle(tmp_path, names, want):
    for n in names:
        os.makedirs(tmp_path / n)
    (tmp_path / "step-file-not-dir").write_text("x")
    ref = ock.find_latest(str(tmp_path))
    got = find_latest_checkpoint(str(tmp_path))
    assert ref == got
    assert (None if got is None else os.path.basename(got)) == want


def test_find_latest_missing_dir(tmp_path):
    """CheckpointTests.FindLatest_ReturnsNull_WhenMissingOrEmpty (CheckpointTests.cs:73-86)."""
    assert find_latest_checkpoint(str(tmp_path / "missing")) is None
    assert ock.find_latest(str(tmp_path / "missing")) is None
    assert find_latest_checkpoint(None) is None


def test_decay_rule_on_reference_names():
    """Only biases escape weight decay: 'RmsNormLayer.weight' does not contain 'norm.weight'."""
    c = ModelConfig(n_layers=1, d_model=64, n_heads=2, n_kv_heads=1, head_dim=32, ffn_dim=96, vocab=64, batch=1,
                    seq=16, qk_norm=1, use_bias=1)
    shapes = {}

    def get(name, shape):
        shapes[name] = shape
        return np.zeros(shape, np.float32)

    names = [n for n, _ in ock.reference_params(c, get)]
    decayed = {n: ock.should_decay(n) for n in names}
    assert not decayed["q_proj.bias"] and not decayed["down_proj.bias"]
    assert decayed["RmsNormLayer.weight"] and decayed["EmbeddingTable.weight"] and decayed["q_proj.weight"]
    assert all(decayed[n] == (not n.endswith(".bias")) for n in names)
    assert ock.should_decay("lora.a") and ock.should_decay("lora.b")
    # the names the rule exempts are matched case-insensitively
    assert not ock.should_decay("LayerNorm.Weight") and not ock.should_decay("Attn.BIAS")
