"""Reader of the reference's activation dumps (moe_rocm.dump; model/layer.rs:1036-1083)."""
import json

import numpy as np
import pytest

import dump_writer as DW
from moe_rocm import dump as D


def _dump(tmp_path, H=64, k=3, E=8, calls=((3,), (2,))):
    rng = np.random.default_rng(1)
    DW.write_meta(tmp_path, H, k, E, 2)
    rows = {0: [], 2: []}
    for layer in (0, 2):
        for (n,) in calls:  # appended call by call, as the reference does per forward
            h = rng.standard_normal((n, H)).astype(np.float32)
            i = np.stack([rng.choice(E, k, replace=False) for _ in range(n)]).astype(np.uint32)
            w = rng.uniform(0, 1, (n, k)).astype(np.float32)
            DW.append(tmp_path, layer, h, i, w)
            rows[layer].append((h, i, w))
    return rows


def test_round_trip_of_appended_calls(tmp_path):
    rows = _dump(tmp_path)
    meta = D.read_meta(tmp_path)
    assert meta == {"hidden_dim": 64, "top_k": 3, "n_experts": 8, "n_layers": 2}
    assert json.loads((tmp_path / "meta.json").read_text()) == meta
    assert D.layers_present(tmp_path) == [0, 2]
    for layer in (0, 2):
        dl = D.read_layer(tmp_path, layer, meta)
        assert dl.n_tokens == 5
        assert np.array_equal(dl.hidden, np.concatenate([r[0] for r in rows[layer]]))
        assert np.array_equal(dl.idx, np.concatenate([r[1] for r in rows[layer]]))
        assert np.array_equal(dl.w.view(np.uint32), np.concatenate([r[2] for r in rows[layer]]).view(np.uint32))


def test_byte_layout_is_the_references(tmp_path):
    DW.write_meta(tmp_path, 4, 2, 8, 1)
    DW.append(tmp_path, 7, np.array([[1.0, -2.0, 0.5, 3.0]], np.float32), np.array([[5, 1]], np.uint32),
              np.array([[0.75, 0.25]], np.float32))
    assert (tmp_path / "layer_07_hidden.bin").read_bytes() == bytes.fromhex("0000803f000000c00000003f00004040")
    assert (tmp_path / "layer_07_routing.bin").read_bytes() == bytes.fromhex("05000000010000000000403f0000803e")
    dl = D.read_layer(tmp_path, 7)
    assert dl.idx.tolist() == [[5, 1]] and dl.w.tolist() == [[0.75, 0.25]]


def test_malformed_dumps_are_refused(tmp_path):
    _dump(tmp_path)
    with open(tmp_path / "layer_00_routing.bin", "ab") as f:
        f.write(b"\x00" * 5)  # a torn record
    with pytest.raises(ValueError, match="whole number"):
        D.read_layer(tmp_path, 0)
    with open(tmp_path / "layer_02_hidden.bin", "ab") as f:
        f.write(b"\x00" * 256)  # one more hidden row than routing records
    with pytest.raises(ValueError, match="hidden rows but"):
        D.read_layer(tmp_path, 2)
    (tmp_path / "meta.json").write_text('{"hidden_dim":64,"top_k":3,"n_layers":2}')
    with pytest.raises(ValueError, match="n_experts"):
        D.read_meta(tmp_path)
