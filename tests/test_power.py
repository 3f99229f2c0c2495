"""Host logic of the board-power sampler (ferret_amd/power.py) on a fake hwmon tree."""
import os
import time

import pytest
import torch

from ferret_amd import power


def _card(root, card, pci, name, microwatts):
    dev = root / "pci" / pci
    hw = dev / "hwmon" / f"hwmon{card[-1]}"
    hw.mkdir(parents=True)
    (hw / name).write_text(f"{microwatts}\n")
    (root / card).mkdir()
    os.symlink(dev, root / card / "device")
    return hw / name


def test_pick_power_file_by_pci_address(tmp_path):
    a = _card(tmp_path, "card0", "0000:05:00.0", "power1_average", 1_000_000)
    b = _card(tmp_path, "card1", "0000:15:00.0", "power1_input", 2_000_000)
    g = str(tmp_path / "card*" / "device" / "hwmon" / "hwmon*")
    real = lambda d: {k: os.path.realpath(v) for k, v in d.items()}
    assert real(power.power_files(g)) == {"card0": str(a), "card1": str(b)}
    card, path = power.pick_power_file("05:00.0", g)
    assert (card, os.path.realpath(path)) == ("card0", str(a))
    card, path = power.pick_power_file("15:00.0", g)
    assert (card, os.path.realpath(path)) == ("card1", str(b))
    # two cards and no address (or an unknown one): no guess
    assert power.pick_power_file(None, g) is None
    assert power.pick_power_file("99:00.0", g) is None


def test_pick_power_file_single_card_and_average_first(tmp_path):
    hw = tmp_path / "pci" / "0000:05:00.0" / "hwmon" / "hwmon3"
    hw.mkdir(parents=True)
    (hw / "power1_input").write_text("5\n")
    (hw / "power1_average").write_text("7\n")
    (tmp_path / "card0").mkdir()
    os.symlink(tmp_path / "pci" / "0000:05:00.0", tmp_path / "card0" / "device")
    g = str(tmp_path / "card*" / "device" / "hwmon" / "hwmon*")
    card, path = power.pick_power_file(None, g)
    assert (card, os.path.realpath(path)) == ("card0", str(hw / "power1_average"))
    assert power.pick_power_file(None, str(tmp_path / "none*")) is None


def test_sampler_mean_skips_the_ramp(tmp_path):
    f = tmp_path / "power1_average"
    f.write_text("100000000\n")  # 100 W
    with power.PowerSampler(str(f), interval=0.005) as s:
        time.sleep(0.1)
        f.write_text("1000000000\n")  # 1000 W
        time.sleep(0.4)
    assert len(s.samples) >= 10
    assert s.samples[0] == pytest.approx(100.0)
    summ = s.summary(skip=0.5)
    assert summ["max_w"] == pytest.approx(1000.0)
    assert summ["mean_w"] > 900.0


def test_sampler_without_a_reading():
    with power.PowerSampler(None) as s:
        pass
    assert s.summary() is None


def test_tile_subset_classes():
    t = torch.tensor([[0, 0, 128], [0, 128, 40], [1, 168, 128], [2, 296, 7], [0, 0, 0]], dtype=torch.int32)
    assert power.tile_subset(t, 4, 128, "full").tolist() == [[0, 0, 128], [1, 168, 128]]
    assert power.tile_subset(t, 4, 128, "partial").tolist() == [[0, 128, 40], [2, 296, 7]]
    assert power.tile_subset(t, 4, 128, "all").shape[0] == 4  # rows past ntiles are not tiles
    with pytest.raises(ValueError):
        power.tile_subset(t, 4, 128, "hot")
