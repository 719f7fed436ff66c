"""Checkpoint save / load of the resident engine against the reference's file format.

The engine writes model.bin / optimizer.bin / meta.json on the device's behalf; the oracle reader
(a restatement of Checkpoint.cs and AdamW.SaveState) checks names, order, [In, Out] layouts and
the bits of every tensor.  Resuming from a checkpoint must continue training bit for bit."""
import json
import os
import re

import numpy as np
import pytest
import torch

from oracle import checkpoint as ock
from sharpmind_amd import SmHipError
from sharpmind_amd.engine import Engine, next_token_labels
from sharpmind_amd.model import PREC_BF16, PREC_FP32, QTYPE_Q8_0, ModelConfig

pytestmark = pytest.mark.gpu

FULL = ModelConfig(n_layers=2, d_model=128, n_heads=4, n_kv_heads=2, head_dim=32, ffn_dim=192, vocab=256, batch=2,
                   seq=64, rope_theta=1e4, rope_neox=0, qk_norm=1, use_bias=1, precision=PREC_FP32)
LORA = ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                   seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=8,
                   lora_alpha=16.0, precision=PREC_BF16)


def _batch(c, dev, seed):
    ids = torch.from_numpy(np.random.default_rng(seed).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    return ids, next_token_labels(ids, c.seq)


def _engine(c, seed):
    eng = Engine(c, lr=1e-3, weight_decay=0.1, max_grad_norm=1.0)
    eng.init_synthetic(seed)
    return eng


def _train(eng, c, dev, steps, seed0=100):
    for i in range(steps):
        ids, labels = _batch(c, dev, seed0 + i)
        eng.step(ids, labels)
    torch.cuda.synchronize()


def _ref(eng, c, state=None):
    return ock.reference_params(c, lambda n, s: eng.get(n, s, state=state))


@pytest.mark.parametrize("c", [FULL, LORA], ids=["full_fp32", "lora_bf16_q8"])
def test_save_matches_reference_format(dev, tmp_path, c):
    eng = _engine(c, 1)
    _train(eng, c, dev, 2)
    eng.save_checkpoint(tmp_path, step=2, loss=1.5, note="unit")
    want = _ref(eng, c)
    got = ock.read_model_bin(str(tmp_path / "model.bin"))
    assert [n for n, _, _ in got] == [n for n, _ in want]
    for (n, dims, data), (_, w) in zip(got, want):
        assert dims == w.shape, n
        assert np.array_equal(data, w), n
    step, lr, ms, vs = ock.read_optimizer_bin(str(tmp_path / "optimizer.bin"), [w.size for _, w in want])
    assert step == 2 and lr == np.float32(1e-3)
    for (n, wm), (_, wv), m, v in zip(_ref(eng, c, "m"), _ref(eng, c, "v"), ms, vs):
        assert np.array_equal(m, wm.ravel()) and np.array_equal(v, wv.ravel()), n
    meta = json.loads((tmp_path / "meta.json").read_text())
    assert meta["step"] == 2 and meta["loss"] == 1.5 and meta["note"] == "unit" and meta["paramCount"] == len(want)
    assert re.fullmatch(r"\d{4}-\d\d-\d\dT\d\d:\d\d:\d\d\.\d{7}Z", meta["savedUtc"])
    eng.close()


@pytest.mark.parametrize("c", [FULL, LORA], ids=["full_fp32", "lora_bf16_q8"])
def test_resume_continues_bit_for_bit(dev, tmp_path, c):
    """Train 2 steps, save, load into an engine with other weights (LoRA: same frozen base,
    which checkpoints do not hold), then one more step on both: identical parameters and state."""
    a = _engine(c, 1)
    _train(a, c, dev, 2)
    a.save_checkpoint(tmp_path, step=2, loss=float("nan"))
    b = _engine(c, 1 if c.lora_rank else 9)
    if c.lora_rank:
        _train(b, c, dev, 1, seed0=500)  # different adapters and optimizer state
    step, loss = b.load_checkpoint(tmp_path)
    assert step == 2 and np.isnan(loss)
    for state in (None, "m", "v"):
        for (n, wa), (_, wb) in zip(_ref(a, c, state), _ref(b, c, state)):
            assert np.array_equal(wa, wb), (state, n)
    _train(a, c, dev, 1, seed0=200)
    _train(b, c, dev, 1, seed0=200)
    for (n, wa), (_, wb) in zip(_ref(a, c), _ref(b, c)):
        assert np.array_equal(wa, wb), n
    a.close()
    b.close()


def test_load_reference_written_checkpoint(dev, tmp_path):
    """A checkpoint written by the format restatement, with a tensor this model lacks."""
    c = FULL
    eng = _engine(c, 3)
    rng = np.random.default_rng(0)
    params = [(n, rng.standard_normal(w.shape).astype(np.float32)) for n, w in _ref(eng, c)]
    ms = [rng.standard_normal(w.size).astype(np.float32) for _, w in params]
    vs = [np.abs(rng.standard_normal(w.size)).astype(np.float32) for _, w in params]
    ock.save(str(tmp_path), [("position_embedding", np.ones((4, 3), np.float32))] + params,
             optimizer=(99, 2e-4, [np.zeros(12, np.float32)] + ms, [np.zeros(12, np.float32)] + vs), step=7,
             loss=0.75, note=None)
    # the optimizer state is positional (LoadState reads m, v per optimizer parameter in order), so
    # write it again without the extra tensor
    ock.write_optimizer_bin(str(tmp_path / "optimizer.bin"), 99, 2e-4, ms, vs)
    step, loss = eng.load_checkpoint(tmp_path)
    assert step == 7 and loss == 0.75
    for (n, w), (_, g) in zip(params, _ref(eng, c)):
        assert np.array_equal(w, g), n
    for m, (n, g) in zip(ms, _ref(eng, c, "m")):
        assert np.array_equal(m, g.ravel()), n
    eng.close()


def test_load_shape_mismatch_is_an_error(dev, tmp_path):
    c = FULL
    eng = _engine(c, 3)
    before = _ref(eng, c)
    bad = [(n, np.zeros(w.size + (1 if n == "o_proj.weight" else 0), np.float32)) for n, w in before]
    ock.save(str(tmp_path), bad)
    with pytest.raises(SmHipError) as ei:
        eng.load_checkpoint(tmp_path)
    msg = str(ei.value)
    assert "o_proj.weight" in msg and str(c.q_dim * c.d_model + 1) in msg and str(c.q_dim * c.d_model) in msg
    for (n, w), (_, g) in zip(before, _ref(eng, c)):  # nothing was written to the device
        assert np.array_equal(w, g), n
    eng.close()


def test_load_without_optimizer_keeps_state(dev, tmp_path):
    c = FULL
    a = _engine(c, 1)
    _train(a, c, dev, 1)
    a.save_checkpoint(tmp_path, step=1)
    b = _engine(c, 2)
    b.load_checkpoint(tmp_path, optimizer=False)
    for (n, wa), (_, wb) in zip(_ref(a, c), _ref(b, c)):
        assert np.array_equal(wa, wb), n
    for n, m in _ref(b, c, "m"):
        assert not m.any(), n
    a.close()
    b.close()


def test_save_without_optimizer(dev, tmp_path):
    eng = _engine(FULL, 1)
    eng.save_checkpoint(tmp_path / "ck", optimizer=False, note='quote " and \\ slash')
    assert sorted(os.listdir(tmp_path / "ck")) == ["meta.json", "model.bin"]
    meta = json.loads((tmp_path / "ck" / "meta.json").read_text())
    assert meta["note"] == 'quote " and \\ slash' and meta["loss"] is None and meta["step"] == 0
    eng.close()
