"""libinfer_calib.so, the measurement aids bench.py reads its floors from
(csrc/calibration.hip): the streaming read covers exactly the bytes it is
given, through both its four-load loop and its tail, and writes nothing
else; the empty kernel launches."""
import pytest

pytestmark = pytest.mark.gpu

SENTINEL = 0x9E3779B9 - (1 << 32)  # the int32 whose presence makes the kernel write its sink


@pytest.mark.parametrize("words, at, blocks", [
    (1 << 20, (1 << 20) - 1, 64),    # last word: the tail loop of the last thread
    (1 << 20, 12345, 64),            # inside the four-load loop
    (1 << 20, 0, 1),                 # one workgroup walks everything
    (4, 3, 2048),                    # one 16-byte chunk, most threads idle
])
def test_stream_read_covers_exactly_its_bytes(dev, words, at, blocks):
    import torch
    import calibration_hip as cal
    print(f"stream_read words={words} at={at} blocks={blocks}", flush=True)
    data = torch.zeros(words, dtype=torch.int32, device=dev)
    data[at] = SENTINEL
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    cal.stream_read(data, sink, blocks)
    torch.cuda.synchronize()
    assert int(sink.item()) == SENTINEL, "the sentinel's chunk was not read"
    # the same buffer without the sentinel's chunk: nothing is written
    sink.zero_()
    chunk = at // 4
    if chunk > 0:
        cal.stream_read(data, sink, blocks, nbytes=16 * chunk)
        torch.cuda.synchronize()
        assert int(sink.item()) == 0, "read past nbytes"


def test_empty_kernel_launches(dev):
    import torch
    import calibration_hip as cal
    cal.empty(608)
    torch.cuda.synchronize()


def test_cu_probes_run_and_time_their_loops(dev):
    """Every compute-unit probe runs to completion on a few workgroups and
    reports a positive loop time on both clocks; a longer loop takes
    longer."""
    import torch
    import calibration_hip as cal
    cycles = torch.zeros(2 * 4, dtype=torch.int64, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    src = torch.ones(1 << 18, dtype=torch.int32, device=dev)  # 1 MiB
    for name in cal.CU_PROBES:
        for threads in (256, 512):
            spans = []
            for iters in (4, 64):
                print(f"cu_probe {name} threads={threads} iters={iters}", flush=True)
                cycles.zero_()
                cal.cu_probe(name, 4, threads, iters, cycles, sink, src)
                torch.cuda.synchronize()
                c = cycles.view(4, 2).cpu()
                assert bool((c > 0).all()), (name, threads, iters, c)
                spans.append(int(c[:, 0].min()))
            assert spans[1] > spans[0], (name, threads, spans)
