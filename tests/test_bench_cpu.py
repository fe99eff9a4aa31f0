"""CPU checks of bench.py's input recipes and baseline helpers (no GPU)."""
import numpy as np
import pytest
import torch

import bench


def test_student_t_recipe_quantiles():
    """z / sqrt(chi2_3 / 3) has the Student-t(3) distribution: its empirical
    quantiles match scipy's t(3) quantiles."""
    from scipy import stats
    x = bench._student_t((1 << 20,), torch.Generator().manual_seed(7)).numpy()
    for p in (0.5, 0.75, 0.9, 0.975, 0.995):
        want = stats.t.ppf(p, 3)
        got = np.quantile(x, p)
        assert abs(got - want) < 0.03 * max(1.0, want), (p, got, want)
    # the same seed gives the same draw
    y = bench._student_t((1 << 20,), torch.Generator().manual_seed(7)).numpy()
    np.testing.assert_array_equal(x, y)


def test_cpu_info_fields():
    info = bench.cpu_info()
    assert info["affinity_cores"] >= 1 and info["torch_threads"] >= 1
    assert isinstance(info["cpu_model"], str) and info["cpu_model"]


def test_port_chunk_bytes_match_oracle():
    """The worker function of the all-cores tier codes a chunk exactly as the
    single-thread tier does (same algorithmic byte count)."""
    from oracle import oracle as O
    t = torch.randn(1, 2, 256, 128, generator=torch.Generator().manual_seed(3)).half().numpy()
    sc = O.cache_scales(O.head_sigma2(t.astype(np.float32)), 4)[0]
    ch = O.compress_chunk(t, 4, scales_f32=sc)
    assert bench._port_chunk((t, sc, 4)) == 4 * t.size + 2 * ch.compressed_bytes


def test_gpus_above_one_refused(monkeypatch, capsys):
    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "one GPU" in capsys.readouterr().err
