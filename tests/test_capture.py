"""Host side of the real-capture path: the capture file format of
AttentionLayer.maybeCapture (Sources/H3Modules/DiTBlock.swift:226-254) and
the axial topology's counted density (AxialTopology.swift:139-170)."""
import numpy as np
import pytest
import torch


def test_capture_names_round_trip():
    from h3hip.capture import capture_name, parse_capture_name
    assert capture_name(3, 0.5) == "qkv_block03_p0.50.safetensors"
    assert capture_name(49, 0.875) == "qkv_block49_p0.88.safetensors"
    assert parse_capture_name("/x/qkv_block24_p0.31.safetensors") == (24, 0.31)
    assert parse_capture_name("qkv_block24.safetensors") is None
    assert parse_capture_name("notes.txt") is None


def test_save_and_load_round_trip_to_head_major(tmp_path):
    from h3hip.capture import capture_name, list_captures, load_qkv, save_qkv
    g = torch.Generator().manual_seed(5)
    S, H, D = 300, 3, 128
    q, k, v = (torch.randn((S, H, D), generator=g).to(torch.bfloat16) for _ in range(3))
    save_qkv(str(tmp_path / capture_name(7, 0.5)), q, k, v)
    save_qkv(str(tmp_path / capture_name(2, 0.75)), q, k, v)
    (tmp_path / "other.bin").write_bytes(b"x")
    files = list_captures(str(tmp_path))
    assert [f.rsplit("/", 1)[1] for f in files] == [capture_name(2, 0.75), capture_name(7, 0.5)]
    qh, kh, vh, s = load_qkv(files[1], device="cpu")
    assert s == S and qh.shape == (H, 384, D) and qh.dtype == torch.bfloat16
    assert torch.equal(qh[:, :S], q.transpose(0, 1)) and torch.equal(vh[:, :S], v.transpose(0, 1))
    assert torch.all(kh[:, S:] == 0)


def test_fp32_captures_are_narrowed_to_bf16(tmp_path):
    from h3hip.capture import load_qkv, save_qkv
    x = torch.randn((130, 1, 128))
    save_qkv(str(tmp_path / "qkv_block00_p0.50.safetensors"), x, x, x)
    q, _, _, _ = load_qkv(str(tmp_path / "qkv_block00_p0.50.safetensors"), device="cpu")
    assert torch.equal(q[0, :130], x[:, 0].to(torch.bfloat16))


def test_malformed_captures_are_refused(tmp_path):
    from safetensors.torch import save_file
    from h3hip.capture import load_qkv, save_qkv
    save_file({"q": torch.zeros(4, 1, 128), "k": torch.zeros(4, 1, 128)}, str(tmp_path / "a.st"))
    with pytest.raises(ValueError, match="q, k and v"):
        load_qkv(str(tmp_path / "a.st"), device="cpu")
    save_file({"q": torch.zeros(4, 1, 128), "k": torch.zeros(5, 1, 128), "v": torch.zeros(4, 1, 128)},
              str(tmp_path / "b.st"))
    with pytest.raises(ValueError, match="shape"):
        load_qkv(str(tmp_path / "b.st"), device="cpu")
    with pytest.raises(ValueError):
        save_qkv(str(tmp_path / "c.st"), torch.zeros(4, 1, 128), torch.zeros(4, 2, 128),
                 torch.zeros(4, 1, 128))


@pytest.mark.parametrize("prefix,frames,h,w,lm", [
    (7, 5, 3, 4, [0, 4]), (0, 6, 4, 5, [0, 2, 5]), (30, 9, 5, 6, [0, 4, 8]), (12, 4, 3, 3, [0, 1, 2, 3]),
])
def test_axial_token_density_matches_the_oracle(orc, prefix, frames, h, w, lm):
    """The closed form against the oracle's closed form and its pair count."""
    from h3hip import axial_token_density
    r = orc.Rule(orc.RULE_AXIAL, prefix + frames * h * w, tile=1, prefix_len=prefix, frames=frames,
                 height=h, width=w, landmarks=lm)
    d = axial_token_density(prefix, frames, h, w, lm)
    assert abs(d - orc.axial_density_closed(r)) < 1e-12
    assert abs(d - orc.token_density_counted(r)) < 1e-9


def test_axial_density_at_the_production_shape(orc):
    """864x480x124: 746 prefix rows, 37x15x27, landmarks [0, 18, 36]."""
    from h3hip import axial_token_density
    from h3hip import configs as C
    sh = C.AXIAL_H3
    kw = sh.oracle_rule_kwargs()
    assert kw["landmarks"] == [0, 18, 36] and sh.seq_len == 15731
    d = axial_token_density(sh.prefix_len, sh.frames, sh.height, sh.width, kw["landmarks"])
    r = orc.Rule(orc.RULE_AXIAL, sh.seq_len, tile=1, prefix_len=746, frames=37, height=15, width=27,
                 landmarks=[0, 18, 36])
    assert abs(d - orc.axial_density_closed(r)) < 1e-12
    assert 0.18 < d < 0.20


def test_memory_plan_drops_the_quadratic_term(h3):
    """MemoryPlan.swift:105-118: a backend that never materialises scores removes
    the quadratic term; at H3's S = 15,731 that is 7.2 GB of the 32.3 GB estimate,
    and the backend's own residents (two outputs per block for 50 blocks, the plan) stay linear."""
    from h3hip.backend import H3HIPBackend, SDPABackend, h3hip_resident_bytes, \
        sampling_activation_bytes
    S = 15731
    dense = sampling_activation_bytes(S, SDPABackend.materialises_scores)
    sparse = sampling_activation_bytes(S, H3HIPBackend.materialises_scores)
    assert dense - sparse == int(2.9e1 * S * S) or abs(dense - sparse - 2.9e1 * S * S) < 2
    assert sparse == int(1.6e6 * S)
    # The reference's fitted point: 53.1 GB at S = 20,392 with the dense backend.
    assert abs(sampling_activation_bytes(20392) / 1e9 - 44.7) < 0.1
    res = h3hip_resident_bytes(S, 56, 50, nnz=10815, n_tiles=123)
    assert res < 24e9 and h3hip_resident_bytes(2 * S, 56, 50, 10815, 246) < 2.01 * res
