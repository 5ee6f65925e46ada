"""Host logic of the T-chunked driver (snn_compiler/nn/chunked.py:31-79), on
the CPU: chunk boundaries, the state hand-over, the ragged last chunk and the
single-call case.  The driver is checked with a forward function that runs
the oracle's LIF recurrence and carries its membrane, so chunked spikes must
equal one pass exactly; the HIP stateful neuron under the same driver is
covered by test_gpu_lif."""
import pytest
import torch

from snnk.nn import run_chunked, ChunkedForward
from oracle import neurons as on


def _lif_forward(calls):
    def fn(x, state):
        calls.append((x.shape[0], state is None))
        s, v, _ = on.lif_multistep(x, neuron="lif", tau=2.0, v_init=state)
        return s, v
    return fn


@pytest.mark.parametrize("chunk", [1, 3, 4, 10, 11, 50])
def test_run_chunked_matches_single_pass(chunk):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(10, 2, 3, 4, generator=g) * 1.5
    ref, _, _ = on.lif_multistep(x, neuron="lif", tau=2.0)
    calls = []
    out = run_chunked(_lif_forward(calls), x, chunk_t=chunk)
    assert torch.equal(out, ref)
    sizes = [c for c, _ in calls]
    assert sum(sizes) == 10 and all(c == min(chunk, 10) for c in sizes[:-1])
    assert [first for _, first in calls] == [True] + [False] * (len(calls) - 1)


def test_chunked_forward_wrapper_and_errors():
    class Net(torch.nn.Module):
        def forward_chunked(self, x, state):
            n = 0 if state is None else state
            return x + n, n + x.shape[0]

        def forward(self, x):
            raise AssertionError("the wrapper must use forward_chunked")

    x = torch.zeros(7, 1)
    out = ChunkedForward(Net(), chunk_t=3)(x)
    assert out.view(-1).tolist() == [0, 0, 0, 3, 3, 3, 6]
    with pytest.raises(ValueError):
        run_chunked(lambda x, s: (x, s), x, chunk_t=0)
