"""Python restatement of the reference's checkpoint files and AdamW state layout.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the sharpmind_amd package.

Follows SharpMind.Training/Checkpoint.cs (Save :27-82, ReadMeta :90-111, FindLatest :117-134,
ParseStep :138-145, Load :161-237) and Optimizers/AdamW.cs (SaveState :96-105, LoadState
:107-117, ShouldDecay :119-125, default no-decay names :38-41).  The parameter list of the
reference's training model (names, order, [In, Out] weight shapes) is restated from
Transformer.cs:239-260, TransformerBlock.cs:52-66, AttentionLayer.cs:425-433,
FFnLayer.cs:317-327, Linearlayer.cs:44-49, NormLayer.cs:126-130, EmbeddingTable.cs:47-50,
ModelFactory.cs:157-190 (tensor shapes) and LoRALayer.cs:94-98 / LoRAAttention.cs:61-67 /
LoRAFFN.cs:24-29 (adapter order).
"""
import json
import os
import struct

import numpy as np

NO_DECAY = ("bias", "norm.weight", "layernorm.weight")  # AdamW.cs:38-41


def should_decay(name, no_decay=NO_DECAY):
    """AdamW.ShouldDecay (AdamW.cs:119-125): ordinal-ignore-case substring test."""
    low = name.lower()
    return not any(nd.lower() in low for nd in no_decay)


# ------------------------------------------------------------------ files
def write_model_bin(path, params):
    """params: [(name, float32 array)] in parameter-list order (Checkpoint.cs:41-58)."""
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(params)))
        for name, a in params:
            nb = name.encode("utf-8")
            f.write(struct.pack("<i", len(nb)))
            f.write(nb)
            a = np.asarray(a, dtype=np.float32)
            f.write(struct.pack("<i", a.ndim))
            for d in a.shape:
                f.write(struct.pack("<i", d))
            f.write(a.astype("<f4").tobytes())


def read_model_bin(path):
    """[(name, dims, float32 array)] in file order."""
    out = []
    with open(path, "rb") as f:
        (count,) = struct.unpack("<i", f.read(4))
        for _ in range(count):
            (n,) = struct.unpack("<i", f.read(4))
            name = f.read(n).decode("utf-8")
            (rank,) = struct.unpack("<i", f.read(4))
            dims = struct.unpack("<%di" % rank, f.read(4 * rank)) if rank else ()
            cnt = int(np.prod(dims)) if rank else 1
            data = np.frombuffer(f.read(4 * cnt), dtype="<f4").astype(np.float32).reshape(dims)
            out.append((name, tuple(dims), data))
        assert f.read(1) == b"", "trailing bytes in model.bin"
    return out


def write_optimizer_bin(path, step, lr, ms, vs):
    """AdamW.SaveState (AdamW.cs:96-105): int32 step, fp32 lr, then m, v of each parameter."""
    with open(path, "wb") as f:
        f.write(struct.pack("<i", step))
        f.write(struct.pack("<f", lr))
        for m, v in zip(ms, vs):
            f.write(np.asarray(m, np.float32).astype("<f4").tobytes())
            f.write(np.asarray(v, np.float32).astype("<f4").tobytes())


def read_optimizer_bin(path, sizes):
    """(stored step, lr, [m], [v]) for parameters of the given element counts."""
    with open(path, "rb") as f:
        step, = struct.unpack("<i", f.read(4))
        lr, = struct.unpack("<f", f.read(4))
        ms, vs = [], []
        for n in sizes:
            ms.append(np.frombuffer(f.read(4 * n), dtype="<f4").astype(np.float32))
            vs.append(np.frombuffer(f.read(4 * n), dtype="<f4").astype(np.float32))
        assert f.read(1) == b"", "trailing bytes in optimizer.bin"
    return step, lr, ms, vs


def write_meta(directory, step, loss, note, param_count, saved_utc="2000-01-01T00:00:00.0000000Z"):
    """Checkpoint.cs:70-81."""
    meta = {"step": step, "loss": None if np.isnan(loss) else float(loss), "note": note, "savedUtc": saved_utc,
            "paramCount": param_count}
    with open(os.path.join(directory, "meta.json"), "w") as f:
        json.dump(meta, f, indent=2)


def read_meta(directory):
    """Checkpoint.ReadMeta (Checkpoint.cs:90-111): (step, loss, note); defaults without a file."""
    path = os.path.join(directory, "meta.json")
    if not os.path.exists(path):
        return 0, float("nan"), None
    with open(path) as f:
        m = json.load(f)
    loss = m.get("loss")
    return int(m.get("step", 0)), float("nan") if loss is None else float(np.float32(loss)), m.get("note")


def save(directory, params, optimizer=None, step=0, loss=float("nan"), note=None):
    """Checkpoint.Save; optimizer = (adam_step, lr, [m], [v]) or None."""
    os.makedirs(directory, exist_ok=True)
    write_model_bin(os.path.join(directory, "model.bin"), params)
    if optimizer is not None:
        write_optimizer_bin(os.path.join(directory, "optimizer.bin"), *optimizer)
    write_meta(directory, step, loss, note, len(params))


class ShapeMismatch(ValueError):
    pass


def load(directory, params, optimizer=None):
    """Checkpoint.Load: params = [(name, float32 array filled in place)] (Checkpoint.cs:161-237).

    Names match first-in-first-out among repeated names; tensors of unknown names are
    skipped; an element-count mismatch raises.  optimizer: dict that receives
    {"step", "lr", "m", "v"} when optimizer.bin exists (LoadState, AdamW.cs:107-117: the
    stored step is skipped and meta.json's step is used)."""
    if not os.path.isdir(directory):
        raise FileNotFoundError(directory)
    queues = {}
    for i, (name, _) in enumerate(params):
        queues.setdefault(name, []).append(i)
    for name, dims, data in read_model_bin(os.path.join(directory, "model.bin")):
        q = queues.get(name)
        if not q:
            continue
        idx = q.pop(0)
        pname, arr = params[idx]
        if data.size != arr.size:
            raise ShapeMismatch(f"Checkpoint tensor '{name}' has {data.size} elements but the model parameter "
                                f"'{pname}' has {arr.size}.")
        arr.reshape(-1)[:] = data.reshape(-1)
    step, loss, note = read_meta(directory)
    opt_path = os.path.join(directory, "optimizer.bin")
    if optimizer is not None and os.path.exists(opt_path):
        _, lr, ms, vs = read_optimizer_bin(opt_path, [a.size for _, a in params])
        optimizer.update(step=step, lr=lr, m=ms, v=vs)
    return step, loss, note


def _parse_step(name):
    """Checkpoint.ParseStep as written (Checkpoint.cs:138-145): the guard is inverted, so every
    name starting with "step-" parses as 0."""
    if not name or not name.strip():
        return 0
    if name.startswith("step-"):
        return 0
    end = name.find("-", 5)
    num = name[5:] if end < 0 else name[5:end]
    try:
        return int(num)
    except ValueError:
        return 0


def find_latest(directory):
    """Checkpoint.FindLatest (Checkpoint.cs:117-134)."""
    if not directory or not os.path.isdir(directory):
        return None
    best, best_step = None, None
    for name in sorted(os.listdir(directory)):
        full = os.path.join(directory, name)
        if not (name.startswith("step-") and os.path.isdir(full)):
            continue
        st = _parse_step(name)
        if best is None or st > best_step or (st == best_step and name > os.path.basename(best)):
            best, best_step = full, st
    return best


# ------------------------------------------------------------------ the reference's parameter list
def reference_params(c, get):
    """[(reference name, float32 array in the reference layout)] for engine config c.

    get(engine_name, shape) returns an engine tensor (names and layouts of
    sharpmind_amd.model.tensor_specs: weights [Out][In], LoRA A [In, r], B [r, Out])."""
    d, F, V, qd, kvd = c.d_model, c.ffn_dim, c.vocab, c.q_dim, c.kv_dim
    nqkv = qd + 2 * kvd
    out = []
    if not c.lora_rank:
        out.append(("EmbeddingTable.weight", get("emb", (V, d))))
        for l in range(c.n_layers):
            p = f"l{l}."
            wqkv = get(p + "wqkv", (nqkv, d))
            bqkv = get(p + "bqkv", (nqkv,)) if c.use_bias else None
            for name, lo, n in (("q_proj", 0, qd), ("k_proj", qd, kvd), ("v_proj", qd + kvd, kvd)):
                out.append((name + ".weight", np.ascontiguousarray(wqkv[lo:lo + n].T)))
                if c.use_bias:
                    out.append((name + ".bias", bqkv[lo:lo + n].copy()))
            out.append(("o_proj.weight", np.ascontiguousarray(get(p + "wo", (d, qd)).T)))
            if c.use_bias:
                out.append(("o_proj.bias", get(p + "bo", (d,))))
            if c.qk_norm:
                out.append(("RmsNormLayer.weight", get(p + "q_norm", (c.head_dim,))))
                out.append(("RmsNormLayer.weight", get(p + "k_norm", (c.head_dim,))))
            out.append(("wgated_proj.weight", np.ascontiguousarray(get(p + "wgu", (2 * F, d)).T)))
            if c.use_bias:
                out.append(("wgated_proj.bias", get(p + "bgu", (2 * F,))))
            out.append(("down_proj.weight", np.ascontiguousarray(get(p + "wd", (d, F)).T)))
            if c.use_bias:
                out.append(("down_proj.bias", get(p + "bd", (d,))))
            out.append(("RmsNormLayer.weight", get(p + "norm1", (d,))))
            out.append(("RmsNormLayer.weight", get(p + "norm2", (d,))))
        out.append(("RmsNormLayer.weight", get("norm_f", (d,))))
        return out
    r = c.lora_rank
    for l in range(c.n_layers):
        for t in ("q", "k", "v", "o", "gate", "up", "down"):
            In, Out = c.lora_geom(t)
            out.append(("lora.a", get(f"l{l}.lora.{t}.A", (In, r))))
            out.append(("lora.b", get(f"l{l}.lora.{t}.B", (r, Out))))
    return out
