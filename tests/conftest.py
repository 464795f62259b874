import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def layer_c0(pkg, dev):
    """BASELINE config 0 weights: seed 0, Q4_K gate_up and down, bf16 shared expert."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=0, device=dev)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)


@pytest.fixture(scope="session")
def layer_c3(pkg, dev):
    """BASELINE config 3 weights: seed 2, Q4_K gate_up and down, uniform routing."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=2, device=dev)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)


@pytest.fixture(scope="session")
def layer_zipf(pkg, dev):
    """BASELINE config 2 weights: seed 1, Zipf(1.1)-skewed router bias."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=1, device=dev, zipf=True)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)


@pytest.fixture(scope="session")
def layer_q6k(pkg, dev):
    """BASELINE config 4 weights: seed 3, Q4_K gate_up + Q6_K down, Zipf routing."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=3, device=dev, down_fmt=pkg.quant.FMT_Q6_K, zipf=True)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)


@pytest.fixture(scope="session")
def layer_q5k(pkg, dev):
    """The shipped artifact's expert widths: Q4_K gate_up + Q5_K down (seed 5, uniform routing)."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=5, device=dev, down_fmt=pkg.quant.FMT_Q5_K)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)


@pytest.fixture(scope="session")
def layer_artifact(pkg, dev):
    """The shipped artifact's widths all at once: F32 router and scalar shared gate, separate
    Q4_K gate and up records, Q5_K down, Q8_0 shared expert (seed 7, Zipf routing)."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=7, device=dev, down_fmt=pkg.quant.FMT_Q5_K, zipf=True,
                              router_dtype=torch.float32, scalar_gate_dtype=torch.float32,
                              split_gate_up=True, shared_fmt=pkg.quant.FMT_Q8_0)
    torch.cuda.synchronize()
    return lw, O.from_device(lw)
