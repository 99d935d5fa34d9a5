"""The module's "auto" choice between the fused and the composed sequence
paths (host logic, no GPU): the measured crossover of forward + backward
time on MI355X."""
import pytest

from sparc_amd.mixer import fused_preferred


@pytest.mark.parametrize("B,T,width,fused", [
    (8, 4096, 32768, True),    # the headline shape: 2048 chains
    (16, 2048, 24576, True),   # the stack's layer shape
    (8, 4096, 8192, True),     # 512 chains: fused 2.70 ms, composed 3.98 ms
    (5, 2048, 8192, True),     # 320 chains: the crossover
    (4, 2048, 8192, False),    # 256 chains: composed 1.13 ms, fused 1.25 ms
    (1, 4096, 4096, False),    # 32 chains: composed 0.50 ms, fused 2.26 ms
    (1, 65536, 2048, False),   # 16 chains over a long sequence
    (1, 512, 4096, True),      # short sequences are launch-bound: fused
    (1, 1, 4096, True),
])
def test_auto_path_rule(B, T, width, fused):
    assert fused_preferred(B, T, width // 2) is fused
