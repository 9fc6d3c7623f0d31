"""Every form captured in one HIP graph: the plain RMSNorm, the out-of-place
and partial-sum forms, and the quantised outputs (FP8 with a scale per row,
one given scale, per-row scales under a bound that changes between replays,
scales per 128 elements in the column-major layout, MXFP8, MXFP4).  None
allocates or issues a memset, so each replay, with fresh inputs copied into
the captured buffers and eager work and synchronisations between replays,
must give the eager call's bytes exactly.
"""
import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ROWS, HIDDEN, EPS = 300, 4096, 1e-6


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def buffers(ops):
    """Outputs of every form, preallocated (nothing is allocated inside the graph)."""
    h, n = HIDDEN, ROWS
    e = lambda *shape, dt=torch.bfloat16: torch.empty(*shape, dtype=dt, device=DEV)  # noqa: E731
    return {
        "plain": [e(n, h)],
        "out": [e(n, h), e(n, h)],
        "reduce": [e(n, h)],
        "fp8": [e(n, h, dt=torch.float8_e4m3fn), e(n, dt=torch.float32)],
        "fp8_static": [e(n, h, dt=torch.float8_e4m3fn)],
        "fp8_ub": [e(n, h, dt=torch.float8_e4m3fn), e(n, dt=torch.float32)],
        # column-major scales with 4 padding columns, which no call writes
        "fp8_group": [e(n, h, dt=torch.float8_e4m3fn), e(h // 128, n + 4, dt=torch.float32).fill_(-1.0)],
        "mxfp8": [e(n, h, dt=torch.uint8), e(n, h // 32, dt=torch.uint8)],
        "mxfp4": [e(n, h // 2, dt=torch.uint8), e(n, h // 32, dt=torch.uint8)],
    }


FORMS = ("plain", "out", "reduce", "fp8", "fp8_static", "fp8_ub", "fp8_group", "mxfp8", "mxfp4")


def run_form(ops, form, x, r, p1, w, sc, bufs, ub=None):
    """One call of `form` on inputs x, r (p1: the second partial sum; ub: the
    bounded FP8 form's bound, a one-element device tensor)."""
    b = bufs[form]
    if form == "plain":
        ops.rms_norm(b[0], x, w, EPS)
    elif form == "out":
        ops.fused_add_rms_norm_out(b[0], b[1], x, w, r, EPS)
    elif form == "reduce":
        ops.reduce_add_rms_norm(b[0], [x, p1], w, r, EPS)
    elif form == "fp8":
        ops.hp_rms_norm_fp8(b[0], b[1], x, w, r, EPS)
    elif form == "fp8_static":
        ops.hp_rms_norm_fp8_static(b[0], sc, x, w, r, EPS)
    elif form == "fp8_ub":
        ops.hp_rms_norm_fp8_ub(b[0], b[1], x, w, r, ub, EPS)
    elif form == "fp8_group":
        ops.hp_rms_norm_fp8_group(b[0], b[1][:, :ROWS].t(), x, w, r, EPS)
    elif form == "mxfp8":
        ops.hp_rms_norm_mx(b[0], b[1], x, w, r, EPS, ops.MXFP8)
    else:
        ops.hp_rms_norm_mx(b[0], b[1], x, w, r, EPS, ops.MXFP4)


def snapshot(form, x, r, bufs):
    """The bytes after a call: the form's outputs, then the residual and the
    input (which the forms that only read them must leave as they were)."""
    return [t.clone().view(torch.uint8) for t in bufs[form] + [r, x]]


def fresh(seed):
    x, r, w = make_inputs(ROWS, HIDDEN, torch.bfloat16, seed)
    p1 = make_inputs(ROWS, HIDDEN, torch.bfloat16, seed + 50)[0]
    return x, r, p1, w


def test_every_form_in_one_hip_graph(ops):
    _, _, _, w = fresh(0)
    wd = w.to(DEV)
    sc = torch.tensor([0.02], dtype=torch.float32, device=DEV)
    ub = torch.tensor([2.0], dtype=torch.float32, device=DEV)   # read by the kernel at each replay
    bufs = buffers(ops)
    # captured inputs: one (x, r, second part) per form
    ins = {f: [torch.empty(ROWS, HIDDEN, dtype=torch.bfloat16, device=DEV) for _ in range(3)] for f in FORMS}
    for f in FORMS:
        for t in ins[f]:
            t.normal_()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in FORMS:  # warm-up outside the graph
            run_form(ops, f, *ins[f], wd, sc, bufs, ub)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for f in FORMS:
            run_form(ops, f, *ins[f], wd, sc, bufs, ub)
    eager_bufs = buffers(ops)
    for rep in range(3):
        print("graph replay", rep, flush=True)
        ub.fill_((2.0, 3.0, 1.5)[rep])   # a new bound: the replay reads it from device memory
        data = {}
        for k, f in enumerate(FORMS):
            x, r, p1, _ = fresh(1000 * rep + 10 * k + 1)
            data[f] = (x, r, p1)
            for t, v in zip(ins[f], data[f]):
                t.copy_(v.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = {f: snapshot(f, ins[f][0], ins[f][1], bufs) for f in FORMS}
        for f in FORMS:
            x, r, p1 = (v.to(DEV) for v in data[f])
            run_form(ops, f, x, r, p1, wd, sc, eager_bufs, ub)
            torch.cuda.synchronize()
            want = snapshot(f, x, r, eager_bufs)
            assert len(got[f]) == len(want)
            for j, (a, b) in enumerate(zip(got[f], want)):
                assert torch.equal(a, b), f"replay {rep}, form {f}, tensor {j}"
