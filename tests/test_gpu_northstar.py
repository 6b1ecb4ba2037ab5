"""The benchmarked north-star step itself against the oracle: bench.py's own
runtimes (its default decode workgroups, kernel and merge choices), 4 streams
at 4095 imported positions, both models (talker 28 layers Hq 16 / Hkv 8 D 128;
thinker 30 layers Hq 8 / Hkv 1 D 256, 25 ring-512 sliding + 5 global) on their
two forked streams, one eager step and then replays of the captured step
graph, as bench.py times them. The talker's first and last layers and one
sliding and one global thinker layer hold host-drawn K/V that the oracle
mirrors; every step's outputs of those layers must match the oracle's
attention at max-abs 1e-2, over the fused appends of the same k/v rows that
the bench appends each step. The launches are also checked to take the paths
the bench reports: every talker layer and every global thinker layer on the
MFMA decode, the sliding layers on the VALU kernel."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def test_north_star_step_matches_the_oracle(monkeypatch):
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py"])
    args = bench.parse()
    n, ctx, replays = args.streams, args.ctx, 3
    th_cfg, tk_cfg = bench.THINKER, bench.TALKER
    thinker, talker = bench.build_runtimes(args, ctx + replays + 8, n)
    checked = {"talker": [0, tk_cfg["layers"] - 1], "thinker": [0, th_cfg["pattern"] - 1]}
    assert not bench.thinker_is_global(checked["thinker"][0]) and bench.thinker_is_global(checked["thinker"][1])
    orcs = {
        "talker": O.OracleCache([O.OracleLayer(tk_cfg["hkv"], tk_cfg["d"])] * tk_cfg["layers"], n),
        "thinker": O.OracleCache([O.OracleLayer(th_cfg["hkv"], th_cfg["d"],
                                                0 if bench.thinker_is_global(i) else th_cfg["window"])
                                  for i in range(th_cfg["layers"])], n),
    }
    host = torch.Generator().manual_seed(4096)
    dev = torch.Generator(device="cuda").manual_seed(1)
    for name, rt, cfg in (("talker", talker, tk_cfg), ("thinker", thinker, th_cfg)):
        shape = (1, cfg["hkv"], ctx - 1, cfg["d"])
        for layer in range(cfg["layers"]):
            for s in range(n):
                if layer in checked[name]:
                    k, v = randn_bf16(host, shape), randn_bf16(host, shape)
                    orcs[name].append(s, layer, to_np(k[0]), to_np(v[0]))
                    k, v = k.cuda(), v.cuda()
                else:
                    k = torch.randn(shape, generator=dev, device="cuda").to(torch.bfloat16)
                    v = torch.randn(shape, generator=dev, device="cuda").to(torch.bfloat16)
                rt.import_(s, layer, k, v)
        rt.synchronize()
    models = {"talker": bench.Model(talker, tk_cfg, n, dev, torch.cuda.Stream()),
              "thinker": bench.Model(thinker, th_cfg, n, dev, torch.cuda.Stream())}
    step = bench.Step([models["talker"], models["thinker"]])
    rts = {"talker": talker, "thinker": thinker}

    def check(tag):
        torch.cuda.synchronize()
        for name, model in models.items():
            for layer in checked[name]:
                q, k, v, o = (to_np(t) for t in model.bufs[layer])
                for s in range(n):
                    orcs[name].append(s, layer, k[s], v[s])
                    ref = orcs[name].attend(s, layer, q[s], model.scale)
                    err = float(np.abs(o[s] - ref).max())
                    assert err <= ATOL, f"{tag}: {name} layer {layer} stream {s} at {ctx - 1 + int(tag[-1])}: {err}"

    before = {name: rt.counters()["mfma_decodes"] for name, rt in rts.items()}
    step()  # eager: sizes the workspaces, as bench.py does before capturing
    check("step 1")
    n_global = sum(bench.thinker_is_global(i) for i in range(th_cfg["layers"]))
    assert talker.counters()["mfma_decodes"] - before["talker"] == tk_cfg["layers"]
    assert thinker.counters()["mfma_decodes"] - before["thinker"] == n_global
    for rt in rts.values():
        rt.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rt in rts.values():
        rt.sync_lengths()
    for r in range(replays):
        graph.replay()
        check(f"replay {r + 2}")
    torch.cuda.synchronize()
    for rt in rts.values():
        rt.sync_lengths()
        assert rt.health() == 0
        assert rt.seq_length(n - 1, 0) == ctx - 1 + 1 + replays
