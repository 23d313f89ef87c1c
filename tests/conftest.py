import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "tt-qwen-resident_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rms(t):
    return float(t.double().pow(2).mean().sqrt())


def assert_bf16_output(got, ref):
    """bf16 outputs (attention / GDN o): rtol 2e-2; elements below 2% of the output RMS are held to an
    absolute 2e-2 x RMS instead (relative error is meaningless at zero crossings)."""
    import torch

    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=2e-2, atol=2e-2 * rms(ref))


def assert_state(got, ref):
    """fp32 recurrent state: rtol 1e-4 (absolute floor 1e-4 x RMS for elements near zero)."""
    import torch

    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=1e-4, atol=1e-4 * rms(ref))


def bf16_ulp_mismatch(got, ref):
    """(max difference in bf16 ulps, fraction of elements that differ) of two bf16-valued tensors."""
    import torch

    a = got.cpu().to(torch.bfloat16).view(torch.int16).int()
    b = ref.cpu().to(torch.bfloat16).view(torch.int16).int()
    d = (a - b).abs()
    return int(d.max()), float((d != 0).float().mean())
