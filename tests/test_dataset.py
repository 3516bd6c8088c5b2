"""Host feed (packed token stream, windows, mean CE) through the C ABI, on the
CPU: these entry points do not touch the GPU.

The expected values restate train/dataset.zig (packing: EOS between examples,
none after the last, :76-96 and :130-135; windows: :50-66; numBatches: :42-47;
JSONL skip rules: :116-131) and commands/finetune.zig:256-268 (computeMeanCe)
in a few lines of numpy each, plus the oracle's materialised softmax CE.
"""
import json

import numpy as np
import pytest

import oracle as O
from valkyr_amd import VkhError
from valkyr_amd.dataset import Dataset, mean_ce


def packed_ref(examples, eos):
    out = []
    for i, e in enumerate(examples):
        out += list(e)
        if i + 1 < len(examples):
            out.append(eos)
    return np.array(out, np.uint32)


def test_packing_and_windows():
    ex = [[5, 6, 7], [8], [], [9, 10]]
    d = Dataset.from_examples(ex, n_pos=3, eos_id=2)
    p = packed_ref(ex, 2)
    assert list(p) == [5, 6, 7, 2, 8, 2, 2, 9, 10]
    assert np.array_equal(d.packed(), p)
    assert d.num_batches() == p.size - 3
    for idx in range(d.num_batches()):
        a, b = d.batch(idx)
        assert np.array_equal(a, p[idx:idx + 3]) and np.array_equal(b, p[idx + 1:idx + 4])


def test_short_stream_has_no_batches():
    d = Dataset.from_examples([[1, 2], [3]], n_pos=4, eos_id=0)  # 4 tokens <= n_pos
    assert d.num_batches() == 0
    with pytest.raises(VkhError) as e:
        d.batch(0)
    assert e.value.name == "BatchIndexOutOfRange"


def test_batch_errors():
    d = Dataset.from_examples([list(range(20))], n_pos=8, eos_id=0)
    with pytest.raises(VkhError) as e:
        d.batch(0, n_input=7)
    assert e.value.name == "InputIdsLen"
    with pytest.raises(VkhError) as e:
        d.batch(0, n_target=9)
    assert e.value.name == "TargetIdsLen"
    with pytest.raises(VkhError) as e:
        d.batch(d.num_batches())
    assert e.value.name == "BatchIndexOutOfRange"


def test_batch_seqs_wraps_modulo_num_batches():
    d = Dataset.from_examples([list(range(100, 130))], n_pos=4, eos_id=0)
    nb = d.num_batches()
    a, b = d.batch_seqs(20, 4, 3)
    for s in range(3):
        w = (20 + 4 * s) % nb
        ea, eb = d.batch(w)
        assert np.array_equal(a[4 * s:4 * s + 4], ea) and np.array_equal(b[4 * s:4 * s + 4], eb)


def test_jsonl_skip_rules(tmp_path):
    lines = [
        '{"ids": [1, 2, 3]}',
        '',                                   # empty
        '   \t ',                             # whitespace only
        'not json',                           # does not parse
        '[1, 2]',                             # not an object
        '{"text": "no ids here"}',            # no ids member
        '{"ids": "1 2"}',                     # ids not an array
        '{"ids": [1, -2]}',                   # not a u32
        '{"ids": [1, 2.5]}',                  # not an integer
        '{"ids": [4294967296]}',              # out of range
        '{"ids": [4, 5], "text": "x", "meta": {"ids": [9]}}',
        '  {"ids": []}\r',
        '{"ids": [4294967295]}  ',
        '{"ids": [7], }',                     # trailing comma: does not parse
    ]
    path = tmp_path / "d.jsonl"
    path.write_text("\n".join(lines))
    d = Dataset.from_jsonl(path, n_pos=2, eos_id=0)
    assert list(d.packed()) == [1, 2, 3, 0, 4, 5, 0, 0, 4294967295]


def test_jsonl_empty_dataset(tmp_path):
    path = tmp_path / "e.jsonl"
    path.write_text('\n{"text": "a"}\n\n')
    with pytest.raises(VkhError) as e:
        Dataset.from_jsonl(path, n_pos=2, eos_id=0)
    assert e.value.name == "EmptyDataset"
    with pytest.raises(VkhError) as e:
        Dataset.from_jsonl(tmp_path / "missing.jsonl", n_pos=2, eos_id=0)
    assert e.value.name == "IoError"


def test_jsonl_matches_examples(tmp_path):
    rng = np.random.default_rng(0)
    ex = [rng.integers(0, 50000, rng.integers(1, 40)).tolist() for _ in range(50)]
    path = tmp_path / "r.jsonl"
    path.write_text("\n".join(json.dumps({"ids": e, "n": i}) for i, e in enumerate(ex)) + "\n")
    a = Dataset.from_jsonl(path, n_pos=16, eos_id=151643)
    b = Dataset.from_examples(ex, n_pos=16, eos_id=151643)
    assert np.array_equal(a.packed(), b.packed())
    assert a.num_batches() == b.num_batches()


def test_mean_ce_matches_oracle_and_numpy():
    n, V = 12, 1000
    logits = O.normal(n * V, 5, 3.0)
    tgt = O.ids(n, 6, V)
    ref = O.softmax_ce_loss(logits, tgt, n, V)
    l64 = logits.reshape(n, V).astype(np.float64)
    m = l64.max(1, keepdims=True)
    lse = (m[:, 0] + np.log(np.exp(l64 - m).sum(1)))
    want = float(np.mean(lse - l64[np.arange(n), tgt]))
    got = mean_ce(logits, tgt, V)
    assert abs(got - want) <= 1e-6 * abs(want)
    assert abs(got - ref) <= 1e-5 * abs(ref)
    # a one-hot-saturated row costs ~0; uniform logits cost log V
    assert abs(mean_ce(np.zeros(V, np.float32), np.array([3], np.uint32), V) - np.log(V)) < 1e-6
