"""The module's "auto" choice between the fused and the composed sequence
paths (host logic, no GPU), as measured on MI355X (forward + backward)."""
import pytest

from sparc_amd.mixer import fused_preferred


@pytest.mark.parametrize("B,T,width", [
    (8, 4096, 32768),    # the headline shape: 2048 chains
    (16, 2048, 24576),   # the stack's layer shape
    (8, 4096, 8192),     # 512 chains: fused 1.94 ms, composed 3.50 ms
    (4, 2048, 8192),     # 256 chains: fused 0.63 ms, composed 0.99 ms
    (1, 4096, 4096),     # 32 chains: fused 0.30 ms (time segments), composed 0.60 ms
    (1, 65536, 2048),    # 16 chains over a long sequence: 1.12 against 1.96 ms
    (1, 512, 4096),
    (1, 1, 4096),
])
def test_auto_path_rule(B, T, width):
    """The fused path, with time segments for few chains, measured faster
    than the composed one at every shape (MI355X, bf16, forward + backward)."""
    assert fused_preferred(B, T, width // 2) is True
