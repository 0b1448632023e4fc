"""A MoE layer whose experts live in host memory (an expert pack) and become device-resident on
demand under a Governor-reserved residency ceiling smaller than the layer's expert set: routes are
formed on the device first (vl_moe_route), the selected experts are made resident through the
matvec accelerator (misses staged through pinned slots on its copy stream, least recently used
experts evicted), and the layer runs on the resident copies. Outputs and routes must equal those of
the same layer with every expert resident (same kernels, weights and routes); the oracle checks the
resident layer elsewhere (test_gpu_moe.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import IQ2_XXS, Q8_0
from vastloom_amd import _lib, ops
from vastloom_amd import expert_pack as xp
from vastloom_amd.accel import KIND_VRAM, Governor, default_limits
from vastloom_amd.residency import HostExpert, ResidentMoeLayer
from vastloom_amd.workloads import random_matrix

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def _setup(tmp_path, gt, dt, E=24, H=512, F=256, seed=3):
    rng = np.random.default_rng(seed)
    mats = {e: {"gate": (gt, F, H, random_matrix(rng, gt, F, H, 0.01)),
                "up": (gt, F, H, random_matrix(rng, gt, F, H, 0.01)),
                "down": (dt, H, F, random_matrix(rng, dt, H, F, 0.01))} for e in range(E + 1)}
    xp.write_pack(tmp_path, 3, mats)
    pack = xp.ExpertPack(tmp_path)
    host = [HostExpert.from_pack(pack.experts[e]) for e in range(E + 1)]
    router = torch.from_numpy((rng.standard_normal((E, H)) * 0.05).astype(np.float32))
    return rng, pack, host, router


def _resident_reference(host, gt, dt, H, F, **kw):
    devs = [ops.DeviceExpert(gt, dt, H, F, h.gate, h.up, h.down) for h in host]
    torch.cuda.synchronize()
    for d in devs:
        d.release_staging()
    return ops.MoeLayer(devs[:-1], devs[-1], width=H, intermediate=F, gate_type=gt, down_type=dt, **kw)


@pytest.mark.parametrize("gt,dt", [(IQ2_XXS, IQ2_XXS), (IQ2_XXS, Q8_0)])
def test_resident_layer_matches_fully_resident_layer(tmp_path, gt, dt):
    E, H, F, K = 24, 512, 256, 4
    print(f"[residency] types={gt},{dt} E={E} K={K}", flush=True)
    rng, pack, host, router = _setup(tmp_path, gt, dt, E, H, F)
    kw = dict(top_k=K, semantics=_lib.SEM_DEEPSEEK, routing=_lib.ROUTE_LEARNED,
              score_fn=_lib.SCORE_SIGMOID, route_scale=1.25, router=router)
    ref = _resident_reference(host, gt, dt, H, F, **kw)
    per_expert = sum(ops.matrix_layout(m.ggml_type, m.rows, m.storage_columns)[1] for m in host[0].matrices(1))
    ceiling = 9 * per_expert  # room for one 3-token call's experts, well below all 25
    gov = Governor(default_limits(vram_hard_limit=ceiling + 64 * MiB, staging_hard_limit=64 * MiB))
    layer = ResidentMoeLayer(gov, host[:-1], host[-1], width=H, intermediate=F, gate_type=gt, down_type=dt,
                             maximum_resident_bytes=ceiling, staging_bytes=4 * MiB,
                             minimum_free_vram_after=0, **kw)
    for i in range(14):
        tokens = 1 if i % 3 else 2
        x = torch.from_numpy(rng.standard_normal((tokens, H)).astype(np.float32)).cuda()
        want = ref.forward(x).cpu().numpy()
        got = layer.forward(x).cpu().numpy()
        ids_ref, w_ref = ref.routes(tokens)
        ids, w = layer.routes(tokens)
        assert np.array_equal(ids, ids_ref) and np.array_equal(w.view(np.uint32), w_ref.view(np.uint32))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
        assert gov.snapshot()["reserved"][KIND_VRAM] <= ceiling + 4 * MiB
    s = layer.stats()
    print(f"  uploads {s['uploaded_bytes']} B in {s['upload_ms']:.1f} ms, evicted {s['evicted']}, "
          f"resident {s['resident_matrices']}", flush=True)
    assert s["evicted"] > 0 and s["resident_bytes"] <= ceiling
    layer.close()
    assert gov.snapshot()["reserved"][KIND_VRAM] == 0
    pack.close()


def test_call_beyond_the_ceiling_is_refused(tmp_path):
    E, H, F, K = 24, 512, 256, 6
    rng, pack, host, router = _setup(tmp_path, IQ2_XXS, IQ2_XXS, E, H, F, seed=4)
    per_expert = sum(ops.matrix_layout(m.ggml_type, m.rows, m.storage_columns)[1] for m in host[0].matrices(1))
    gov = Governor(default_limits(vram_hard_limit=256 * MiB, staging_hard_limit=64 * MiB))
    layer = ResidentMoeLayer(gov, host[:-1], host[-1], width=H, intermediate=F, gate_type=IQ2_XXS,
                             down_type=IQ2_XXS, top_k=K, semantics=_lib.SEM_DEEPSEEK,
                             routing=_lib.ROUTE_LEARNED, router=router,
                             maximum_resident_bytes=4 * per_expert, staging_bytes=4 * MiB,
                             minimum_free_vram_after=0)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).cuda()
    with pytest.raises(ValueError):
        layer.forward(x)
    layer.close()
    pack.close()
