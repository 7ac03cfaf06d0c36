"""HIP graph capture of a process's first library call: a prefill.

The first prefill of a process looks up the sigmoid table (constant data in the code object), sets the GEMM
kernels' LDS attribute and creates the side stream of its caller stream.  None of that is stream work, so the
call may be the first one of a process and run under stream capture.  The case runs in a child process whose
inputs are made by torch alone (no library call before the captured one); the graph is replayed three times with
eager library calls and synchronisations between the replays, and every replay must equal the eager result bit
for bit."""
import pytest

from helpers import CHILD_COMMON, run_child

pytestmark = pytest.mark.gpu

PREFILL_CHILD = CHILD_COMMON + r"""
H, I, E, k, T = 4096, 2048, 64, 8, 300
bank = torch_bank(E, H, I)
b = pools.bank_struct(bank)
x = bf16(T, H)
rng = np.random.default_rng(3)
p = 1.0 / np.arange(1, E + 1) ** 1.1
inds = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
counts = np.bincount(inds.reshape(-1), minlength=E)
assert (counts > 64).any() and ((counts > 0) & (counts <= 32)).any()     # wide and narrow tiles both
si = torch.from_numpy(inds).to(dev)
w = torch.rand(T, k, device=dev)
nb = _lib.load().mimo_moe_prefill_workspace_size(T, k, E, H, I)
ws_g = torch.empty(nb, dtype=torch.uint8, device=dev)
ws_e = torch.empty(nb, dtype=torch.uint8, device=dev)
y_g = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
y_e = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
st_g = torch.full((1,), 77, dtype=torch.int32, device=dev)
st_e = torch.full((1,), 77, dtype=torch.int32, device=dev)
torch.cuda.synchronize()
def prefill(y, st, ws):
    _lib.call("mimo_moe_prefill", _lib.ptr(x), T, _lib.ptr(si), _lib.ptr(w), k, b, _lib.ptr(y), _lib.ptr(st),
              _lib.ptr(ws), nb, _lib.stream_ptr())
say("capturing the first prefill of the process")
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    prefill(y_g, st_g, ws_g)
say("captured; eager reference")
prefill(y_e, st_e, ws_e)
torch.cuda.synchronize()
assert int(st_e.item()) == 0
x2 = bf16(T, H)
for rep in range(3):
    y_g.fill_(7.0); st_g.fill_(77)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_g, y_e), f"replay {rep} differs from the eager prefill"
    assert int(st_g.item()) == 0, rep
    x_keep = x.clone(); x.copy_(x2)
    prefill(y_e, st_e, ws_e)                 # eager work between replays (other inputs), then the reference again
    x.copy_(x_keep)
    prefill(y_e, st_e, ws_e)
    torch.cuda.synchronize()
    say(f"replay {rep} ok")
say("PREFILL_FIRST_CALL_OK")
"""


def test_first_prefill_of_a_process_captured():
    run_child(PREFILL_CHILD, "PREFILL_FIRST_CALL_OK")


# More caller streams than the library keeps side streams for (64 per device): the prefills on the later streams
# run both tile launches on their own stream and give the same bits.
MANY_STREAMS_CHILD = CHILD_COMMON + r"""
H, I, E, k, T = 1024, 512, 64, 8, 300
bank = torch_bank(E, H, I)
b = pools.bank_struct(bank)
x = bf16(T, H)
rng = np.random.default_rng(4)
p = 1.0 / np.arange(1, E + 1) ** 1.1
inds = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
counts = np.bincount(inds.reshape(-1), minlength=E)
assert (counts > 64).any() and ((counts > 0) & (counts <= 32)).any()     # wide and narrow tiles both
si = torch.from_numpy(inds).to(dev)
w = torch.rand(T, k, device=dev)
nb = _lib.load().mimo_moe_prefill_workspace_size(T, k, E, H, I)
ws = torch.empty(nb, dtype=torch.uint8, device=dev)
st = torch.full((1,), 77, dtype=torch.int32, device=dev)
def prefill(y):
    _lib.call("mimo_moe_prefill", _lib.ptr(x), T, _lib.ptr(si), _lib.ptr(w), k, b, _lib.ptr(y), _lib.ptr(st),
              _lib.ptr(ws), nb, _lib.stream_ptr())
y_ref = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
prefill(y_ref)
torch.cuda.synchronize()
assert int(st.item()) == 0
streams = [torch.cuda.Stream() for _ in range(70)]
y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
for n, s in enumerate(streams):
    y.fill_(7.0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        prefill(y)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), f"prefill on caller stream {n} differs"
    assert int(st.item()) == 0, n
say(f"{len(streams)} caller streams ok")
say("MANY_STREAMS_OK")
"""


def test_prefill_on_more_streams_than_side_streams():
    run_child(MANY_STREAMS_CHILD, "MANY_STREAMS_OK")
