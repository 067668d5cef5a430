"""Host-side contract of the reference-named loader ``load_resident_moe_layer``
(``runtime/dsv4_direct/ops/marlin_moe.py:270-307``): the checkpoint id must be
a lowercase SHA-256 and the input dtype None or float8_e4m3fn, both refused
with ValueError before any file is read; the TP slice must keep 128-row
blocks whole."""

import pytest
import torch

from gaiban_lite_amd import checkpoint as CK

KW = dict(layer_id=0, rank=0, world_size=1, hidden_size=512, intermediate_size=1024, n_experts=8,
          device=torch.device("cpu"))


@pytest.mark.parametrize("bad", [None, "", "0" * 63, "0" * 65, "0123456789ABCDEF" * 4, "g" * 64, 1234])
def test_checkpoint_id_must_be_lowercase_sha256(tmp_path, bad):
    with pytest.raises(ValueError, match="SHA-256"):
        CK.load_resident_moe_layer(stage_root=tmp_path / "absent", checkpoint_id=bad, **KW)


def test_input_dtype_and_slice_checks(tmp_path):
    sha = "ab" * 32
    with pytest.raises(ValueError, match="marlin_input_dtype"):
        CK.load_resident_moe_layer(stage_root=tmp_path / "absent", checkpoint_id=sha, marlin_input_dtype=torch.int8,
                                   **KW)
    kw = dict(KW, world_size=3)
    with pytest.raises(ValueError):
        CK.load_resident_moe_layer(stage_root=tmp_path / "absent", checkpoint_id=sha, **kw)
    kw = dict(KW, world_size=16)  # 64-row slices break the 128-row FP8 blocks
    with pytest.raises(ValueError, match="block"):
        CK.load_resident_moe_layer(stage_root=tmp_path / "absent", checkpoint_id=sha, **kw)
