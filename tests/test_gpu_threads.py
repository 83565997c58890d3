"""Concurrent calls from several host threads on one GPU.

The binning forks work onto a side stream and joins it back; each calling
thread has its own side stream and events.  Two threads rendering different
scenes at the same time, repeatedly, give exactly the images and lists a
single thread gives (the forward is deterministic)."""

from __future__ import annotations

import threading

import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline

pytestmark = pytest.mark.gpu


def _inputs(scene, device):
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    return (*(t.to(device) for t in scene.params()), cam.rotation_matrix, cam.translation,
            fx, fy, cx, cy, w, h, 16, 0.999, scene.near, scene.far, "gaussian", 0.95)


def test_two_threads_render_like_one(device):
    work = [_inputs(scenes.edge_case_scene(n=3000, sh_degree=3, image_size=(200, 120)), device),
            _inputs(scenes.edge_case_scene(n=5000, sh_degree=1, image_size=(320, 240)), device)]
    expected = []
    for inputs in work:
        out = forward_pipeline(*inputs, record_hits=False)
        torch.cuda.synchronize(device)
        expected.append([t.clone() for t in (out[0], out[1], out[2], out[7], out[8])])
    results = [[], []]
    errors = []

    def run(k):
        try:
            for _ in range(8):
                out = forward_pipeline(*work[k], record_hits=False)
                torch.cuda.synchronize(device)
                results[k].append([t.clone() for t in (out[0], out[1], out[2], out[7], out[8])])
        except Exception as e:  # reported in the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    print("[threads] two threads x 8 forwards", flush=True)
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a rendering thread did not finish"
    assert not errors, errors
    for k in range(2):
        assert len(results[k]) == 8
        for got in results[k]:
            for a, b in zip(got, expected[k]):
                assert torch.equal(a, b)
