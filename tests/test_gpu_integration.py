"""A quantized two-layer model under HIP-graph capture and torch.compile.

Mirrors the reference's integration tests (tests/test_integration.py:14-216): weights
stored as QuantizedTensors, inputs quantized at run time, F.linear on quantized
operands, an activation in between.  Here every layout runs on the hip kernels, and
the activations use the device-side dynamic scale (scale=None), so a captured graph
also replays the amax kernels.
"""
import pytest
import torch
import torch.nn.functional as F

from comfy_kitchen.tensor import QuantizedTensor

pytestmark = pytest.mark.gpu

LAYOUTS = ["TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"]


class TwoLayer(torch.nn.Module):
    def __init__(self, layout: str, in_features=256, hidden=512, out_features=128, seed=0):
        super().__init__()
        g = torch.Generator(device="cuda").manual_seed(seed)
        w1 = (torch.randn(hidden, in_features, device="cuda", generator=g) * 0.05).bfloat16()
        w2 = (torch.randn(out_features, hidden, device="cuda", generator=g) * 0.05).bfloat16()
        self.layout = layout
        self.w1 = QuantizedTensor.from_float(w1, layout)
        self.w2 = QuantizedTensor.from_float(w2, layout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = F.linear(QuantizedTensor.from_float(x, self.layout), self.w1)
        h = F.gelu(h)
        return F.linear(QuantizedTensor.from_float(h, self.layout), self.w2)


def _input(seed, rows=64, cols=256):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(rows, cols, device="cuda", generator=g).bfloat16()


# (rows, in_features, hidden, out_features): 64 rows run the skinny GEMM kernels; 256 rows
# against K = 4096 and 512 outputs split K over a workspace (two launches per GEMM)
SHAPES = [(64, 256, 512, 128), (256, 4096, 512, 128)]


@pytest.mark.parametrize("shape", SHAPES, ids=["skinny", "split_k"])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_graph_capture_replay(layout, shape, hip):
    rows, fin, hidden, fout = shape
    model = TwoLayer(layout, in_features=fin, hidden=hidden, out_features=fout)
    if shape[0] == 256:
        import comfy_kitchen.backends.hip as hb

        fn = ("ckh_scaled_mm_nvfp4_workspace_bytes" if layout == "TensorCoreNVFP4Layout"
              else "ckh_scaled_mm_workspace_bytes")
        assert getattr(hb._lib, fn)(rows, hidden, fin) > 0  # the first GEMM splits K
    x = _input(1, rows, fin)
    with torch.no_grad():
        want = model(x)
        static_x = x.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                model(static_x)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = model(static_x)
        # replays with the program's own eager work and synchronizations in between
        for i in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, want), f"replay {i} differs from eager"
            eager = model(_input(10 + i, rows, fin))
            torch.cuda.synchronize()
            assert eager.shape == want.shape
        # a new input through the same graph
        x2 = _input(2, rows, fin)
        static_x.copy_(x2)
        graph.replay()
        torch.cuda.synchronize()
        want2 = model(x2)
        assert torch.equal(static_out, want2)
        assert not torch.equal(want, want2)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_compile(layout, hip):
    model = TwoLayer(layout)
    x = _input(3)
    with torch.no_grad():
        want = model(x)
        compiled = torch.compile(model)
        runs = [compiled(x).clone() for _ in range(3)]
    assert runs[0].shape == want.shape and runs[0].dtype == want.dtype
    # inductor may round the GELU differently from eager, and a one-ulp change can move
    # a requantized activation to the next code, so the bound is on rel-L2, not bits
    rel = ((runs[0].float() - want.float()).norm() / want.float().norm()).item()
    assert rel <= 2e-2, rel
    for r in runs[1:]:
        assert torch.equal(runs[0], r)
