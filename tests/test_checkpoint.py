"""model.pt checkpoints (the reference's main.py:86-94 layout) read with the weights-only loader."""
import pytest
import torch
import torch.nn.functional as F

from gaussian_splatting.utils.checkpoint import CameraView, load_camera, load_checkpoint, save_camera, save_checkpoint


def reference_layout(n=50, rest=15, degree=3):
    g = torch.Generator().manual_seed(0)
    return {
        "params": {
            "means": torch.randn(n, 3, generator=g), "scales": torch.randn(n, 3, generator=g) - 4,
            "quats": torch.randn(n, 4, generator=g) * 3, "opacities": torch.randn(n, 1, generator=g),
            "sh_dc": torch.randn(n, 1, 3, generator=g), "sh_rest": torch.randn(n, rest, 3, generator=g),
        },
        "active_sh_degree": degree, "iteration": 30000, "test_psnr": 25.5,
    }


def test_reads_the_reference_layout_and_activates_like_gaussian_model(tmp_path):
    state = reference_layout()
    torch.save(state, tmp_path / "model.pt")  # written the way main.py:86-94 writes it
    ckpt = load_checkpoint(tmp_path / "model.pt")
    p = state["params"]
    assert ckpt.n == 50 and ckpt.active_sh_degree == 3 and ckpt.iteration == 30000 and ckpt.test_psnr == 25.5
    assert torch.equal(ckpt.means, p["means"])
    assert torch.equal(ckpt.scales, torch.exp(p["scales"]))
    assert torch.equal(ckpt.quats, F.normalize(p["quats"], dim=-1))
    assert torch.equal(ckpt.opacities, torch.sigmoid(p["opacities"]))
    assert torch.allclose(ckpt.quats.norm(dim=-1), torch.ones(50))


def test_save_then_load_round_trips(tmp_path):
    state = reference_layout(n=7, rest=3, degree=1)
    save_checkpoint(tmp_path / "m.pt", state["params"], 1, 12, 20.0)
    ckpt = load_checkpoint(tmp_path / "m.pt")
    for name, t in state["params"].items():
        assert torch.equal(ckpt.params[name], t)
    assert (ckpt.active_sh_degree, ckpt.iteration, ckpt.test_psnr) == (1, 12, 20.0)


@pytest.mark.parametrize("breakage", ["no_params", "bad_quats", "bad_rest", "degree_too_high"])
def test_rejects_malformed_files(tmp_path, breakage):
    state = reference_layout(rest=3, degree=1)
    if breakage == "no_params":
        del state["params"]
    elif breakage == "bad_quats":
        state["params"]["quats"] = torch.zeros(50, 3)
    elif breakage == "bad_rest":
        state["params"]["sh_rest"] = torch.zeros(50, 4, 3)
    else:
        state["active_sh_degree"] = 2
    torch.save(state, tmp_path / "model.pt")
    with pytest.raises(ValueError):
        load_checkpoint(tmp_path / "model.pt")


class Payload:
    """An arbitrary class: loading an instance would run the unpickler's class lookup."""


def test_refuses_files_that_need_unpickling_code(tmp_path):
    torch.save({"params": {}, "active_sh_degree": 0, "payload": Payload()}, tmp_path / "model.pt")
    with pytest.raises(Exception, match="[Ww]eights only|weights_only|Unsupported"):
        load_checkpoint(tmp_path / "model.pt")


def rotated_view(name="view0"):
    """A camera turned 30 degrees about y, 4 units back: world_to_camera = [R | t]."""
    a = torch.tensor(0.5235987755982988)
    rot = torch.tensor([[torch.cos(a), 0.0, torch.sin(a)], [0.0, 1.0, 0.0], [-torch.sin(a), 0.0, torch.cos(a)]])
    w2c = torch.eye(4)
    w2c[:3, :3] = rot
    w2c[:3, 3] = torch.tensor([0.1, -0.2, 4.0])
    return CameraView(w2c, 300.0, 310.0, 128.5, 95.0, 256, 192, name)


def test_camera_round_trips_and_its_centre_maps_to_the_camera_origin(tmp_path):
    view = rotated_view()
    save_camera(tmp_path / "cam.json", view)
    back = load_camera(tmp_path / "cam.json")
    assert torch.equal(back.world_to_camera, view.world_to_camera)
    assert (back.fx, back.fy, back.cx, back.cy, back.width, back.height, back.name) == \
        (300.0, 310.0, 128.5, 95.0, 256, 192, "view0")
    # The centre is the world point the transform sends to the camera's origin.
    c = torch.cat([back.center, torch.ones(1)])
    torch.testing.assert_close(back.world_to_camera @ c, torch.tensor([0.0, 0.0, 0.0, 1.0]), atol=1e-6, rtol=0)


@pytest.mark.parametrize("breakage", ["missing", "shape", "last_row", "size"])
def test_camera_rejects_malformed_files(tmp_path, breakage):
    import json

    spec = {"world_to_camera": torch.eye(4).tolist(), "fx": 1.0, "fy": 1.0, "cx": 0.5, "cy": 0.5, "width": 8,
            "height": 8}
    if breakage == "missing":
        del spec["fy"]
    elif breakage == "shape":
        spec["world_to_camera"] = torch.eye(3).tolist()
    elif breakage == "last_row":
        spec["world_to_camera"][3][0] = 1.0
    else:
        spec["width"] = 0
    (tmp_path / "cam.json").write_text(json.dumps(spec))
    with pytest.raises(ValueError):
        load_camera(tmp_path / "cam.json")


def test_bench_builds_the_harness_frame_from_a_checkpoint(tmp_path):
    """bench.py --checkpoint/--camera: activated gaussians, the raw quats as the leaf (bench/harness.py:43),
    the checkpoint's SH degree, the camera's pose and intrinsics, features U[0, 1]."""
    import bench

    state = reference_layout(n=40, rest=15, degree=2)
    torch.save(state, tmp_path / "model.pt")
    save_camera(tmp_path / "cam.json", rotated_view())
    wl = bench.checkpoint_workload(tmp_path / "model.pt", tmp_path / "cam.json", 16)
    p = state["params"]
    assert (wl.n, wl.width, wl.height, wl.channels, wl.sh_degree) == (40, 256, 192, 16, 2)
    assert torch.equal(wl.scales, torch.exp(p["scales"])) and torch.equal(wl.opacities, torch.sigmoid(p["opacities"]))
    assert torch.equal(wl.quats, p["quats"])
    assert wl.cam == {"fx": 300.0, "fy": 310.0, "cx": 128.5, "cy": 95.0, "width": 256, "height": 192}
    assert torch.equal(wl.world_to_camera, rotated_view().world_to_camera)
    torch.testing.assert_close(wl.center, rotated_view().center)
    assert wl.features.shape == (40, 16) and float(wl.features.min()) >= 0 and float(wl.features.max()) < 1
