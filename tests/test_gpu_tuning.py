"""Tuned mode on the GPU (memfast/simulator.py:195-347 protocol, grid re-keyed to the
gfx950 kernels' launch parameters in memfast_amd/tuning.py).

Every selected schedule must give the default schedule's output bit for bit; the
cache file is written atomically and revalidated bit for bit by a second
simulator; a corrupt or stale cache file is ignored; candidates whose scratch
exceeds the workspace budget, or whose LDS tier cannot hold a read, are
rejected with a reason.
"""

import json

import pytest
import torch

from memfast_amd import Config, Nonidealities, Simulator, tuning

pytestmark = pytest.mark.gpu

INT8 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
            weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))


def say(*args):
    print("[tuning]", *args, flush=True)


def bits_equal(a, b):
    view = torch.int32 if a.dtype == torch.float32 else torch.int64
    return a.shape == b.shape and torch.equal(a.view(view), b.view(view))


def operands(n, k, o, device, seed=3, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(n, k, generator=gen).to(device)
    b = (torch.randn(k, o, generator=gen) * scale).to(device)
    return a, b


def default_output(cfg, a, b, device):
    return Simulator(cfg, device=device).mm(a, b)


def test_tuned_ideal_selection_cache_and_revalidation(hip_device, tmp_path):
    cfg = Config(**INT8, nonidealities=Nonidealities(write_variation=0.0))
    a, b = operands(512, 1024, 768, hip_device)
    expected = default_output(cfg, a, b, hip_device)
    sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    got = sim.mm(a, b)
    assert bits_equal(got, expected)
    record = sim.report()["selections"][0]
    say("first", {k: record[k] for k in ("kernel", "cache_hit", "selected", "domain_count")})
    assert record["kernel"] == 1 and record["complete"] and not record["cache_hit"]
    assert [c["schedule"]["tile"] for c in record["candidates"]] == ["64x64", "128x64"]
    assert all(c["status"] == "accepted" and c["seconds"] > 0 for c in record["candidates"])
    files = list(tmp_path.iterdir())
    assert [f.name for f in files] == [f"{record['key']}.json"]   # no temporary left over
    content = json.loads(files[0].read_text())
    assert content["complete"] is True and content["selected"] == record["selected"]
    # A second simulator hits the cache, revalidates bit for bit and times nothing.
    again = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    assert bits_equal(again.mm(a, b), expected)
    hit = again.report()["selections"][0]
    assert hit["cache_hit"] and hit["candidates"] == [] and hit["selected"] == record["selected"]
    # A different input shape is a different key.
    again.mm(a[:100], b)
    assert len(list(tmp_path.iterdir())) == 2


def test_tuned_cache_corrupt_or_stale_is_ignored(hip_device, tmp_path):
    cfg = Config(**INT8, nonidealities=Nonidealities(write_variation=0.0))
    a, b = operands(256, 512, 300, hip_device, seed=4)
    first = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    expected = first.mm(a, b)
    path = tmp_path / f"{first.report()['selections'][0]['key']}.json"
    stored = json.loads(path.read_text())
    cases = {
        "corrupt": "{not json",
        "incomplete": json.dumps(dict(stored, complete=False)),
        "foreign schedule": json.dumps(dict(stored, selected=dict(stored["selected"],
                                                                   tile="256x256"))),
        "other fingerprint": json.dumps(dict(stored, fingerprint=dict(stored["fingerprint"],
                                                                      shape=[1, 1]))),
    }
    for name, text in cases.items():
        path.write_text(text)
        sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
        assert bits_equal(sim.mm(a, b), expected), name
        record = sim.report()["selections"][0]
        assert not record["cache_hit"] and len(record["candidates"]) == 2, name
        assert json.loads(path.read_text())["complete"] is True, name   # rewritten


def test_tuned_noisy_split_candidates_under_a_budget(hip_device, tmp_path):
    """256 vectors x 512 x 1024 on 128x128 arrays: 64 blocks, so the automatic schedule
    splits the reads.  A 20 MiB budget holds the 10.5 MB of conductance terms but not a
    split's 16.8 MB of integer totals: the default and every split candidate are rejected
    for the workspace budget, the unsplit read is selected and equals the default mode's
    split output bit for bit (with write and shared read noise and the S-curve ADC)."""
    cfg = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02, read_variation=0.01,
                                                     adc_nonlinearity=0.1))
    a, b = operands(256, 512, 1024, hip_device, seed=5)
    expected = default_output(cfg, a, b, hip_device)
    sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path, workspace_mb=20)
    assert bits_equal(sim.mm(a, b), expected)
    record = sim.report()["selections"][0]
    status = {c["schedule"]["split"]: (c["status"], c.get("reason")) for c in record["candidates"]}
    say("noisy splits", status)
    assert record["kernel"] == 2
    assert status[1][0] == "accepted"
    for split in (0, 2, 4, 8):
        assert status[split] == ("rejected", "workspace budget"), split
    assert record["selected"]["split"] == 1
    # With the default budget every split is feasible and all agree bit for bit.
    roomy = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path / "roomy")
    assert bits_equal(roomy.mm(a, b), expected)
    record = roomy.report()["selections"][0]
    assert all(c["status"] == "accepted" for c in record["candidates"])


@pytest.mark.parametrize("name", ["config5", "four_weight_slices"])
def test_tuned_wide_lds_tiers(hip_device, tmp_path, name):
    """Wide noisy reads (BASELINE config 5's slicing; and four weight slices at 64-row reads,
    32 fragments per read, which the 24-fragment tier cannot hold)."""
    if name == "config5":
        cfg = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                     weight_slice=(1, 1, 2), bw_e=8, adc_bits=(6, 6, 7),
                     nonidealities=Nonidealities(read_variation=0.01, drift_coefficient=0.05,
                                                 drift_time=100.0))
        a, b = operands(128, 512, 256, hip_device, seed=6, scale=0.02)
    else:
        cfg = Config(activation_bits=10, weight_bits=7, input_slice=(1, 1, 4, 4),
                     weight_slice=(1, 2, 2, 2), array_size=(128, 64), rows_per_read=64,
                     adc_bits=8, nonidealities=Nonidealities(write_variation=0.02))
        a, b = operands(130, 300, 130, hip_device, seed=7, scale=0.02)
    expected = default_output(cfg, a, b, hip_device)
    sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    assert bits_equal(sim.mm(a, b), expected)
    record = sim.report()["selections"][0]
    status = {c["schedule"]["tier"]: (c["status"], c.get("reason")) for c in record["candidates"]}
    say(name, status, "selected", record["selected"])
    assert record["kernel"] == 3 and set(status) == {0, 1, 2, 3}
    if name == "config5":
        assert all(state == "accepted" for state, _ in status.values())
    else:
        assert status[1][0] == "rejected" and "LDS tier" in status[1][1]
        assert all(status[t][0] == "accepted" for t in (0, 2, 3))


def test_tuned_layer_reuses_its_selection(hip_device, tmp_path):
    """A tuned layer selects once per input shape and dtype; later reads reuse the schedule
    (no new record) and equal default-mode reads at the same read events."""
    from torch import nn

    from memfast_amd.nn import AnalogLinear

    cfg = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(8)
    source = nn.Linear(384, 200).to(hip_device)
    tuned_sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    tuned = AnalogLinear(source, tuned_sim, name="fc")
    plain = AnalogLinear(source, Simulator(cfg, device=hip_device), name="fc")
    x = torch.randn(96, 384, device=hip_device)
    for _ in range(3):
        assert bits_equal(tuned(x), plain(x))
    assert len(tuned_sim.records) == 1 and tuned._event == plain._event == 3
    assert tuning.read_kernel(cfg, 96, 3, tuned.p) == 2


def test_resources_follow_the_schedule(hip_device):
    """mf_resources_query reports the instance a schedule launches, as the reference reads
    each candidate's own compiled kernel (memfast/simulator.py:230-236): the ideal read's
    64x64 and 128x64 tiles (k_ideal<1,1>, k_ideal<2,1>) and the wide read's LDS tiers."""
    from memfast_amd import hip

    ideal = Config(**INT8, nonidealities=Nonidealities(write_variation=0.0))
    program = hip.program(ideal, 64, 64, hip_device.index)
    tiles = {name: program.resources(ideal, 64, 64, 0, kernel=1,
                                     variant=tuning.schedule_variant(dict(tile=name)))
             for name in tuning.TILES}
    say("ideal tiles", tiles)
    assert tiles["64x64"]["registers"] != tiles["128x64"]["registers"]
    assert tiles["64x64"]["shared"] < tiles["128x64"]["shared"]
    wide = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                  weight_slice=(1, 1, 2), bw_e=8, array_size=(64, 64), rows_per_read=64,
                  adc_bits=(6, 6, 7), nonidealities=Nonidealities(write_variation=0.02))
    program = hip.program(wide, 64, 64, hip_device.index)
    tiers = {tier: program.resources(wide, 64, 64, 0, kernel=3,
                                     variant=tuning.schedule_variant(dict(tier=tier)))
             for tier in tuning.TIERS}
    say("wide tiers", tiers)
    assert tiers[1]["shared"] < tiers[2]["shared"] < tiers[3]["shared"]
    # The automatic tier is the smallest that holds a read (3 weight slices x 2 terms x 4).
    assert program.resources(wide, 64, 64, 0, kernel=3) == tiers[1]
    # The noisy read of at most 32 vectors runs k_noisy_pairs (one wave per weight slice)
    # unless the schedule never splits.
    noisy = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02))
    program = hip.program(noisy, 64, 64, hip_device.index)
    small = program.resources(noisy, 64, 64, 0, kernel=2, batch=32)
    unsplit = program.resources(noisy, 64, 64, 0, kernel=2, batch=32,
                                variant=tuning.schedule_variant(dict(split=1)))
    large = program.resources(noisy, 64, 64, 0, kernel=2, batch=33)
    say("noisy small batch", small, "unsplit", unsplit, "large", large)
    assert small["threads"] == 64 * len(noisy.weight_layout)
    assert unsplit == large and large["threads"] == 256
