"""pk_joint_scan_noalloc (static library scratch, no allocation) against
pk_joint_scan (caller workspace) through the C ABI: two calls in a row on
the same GPU, the second with a smaller joint (fewer rows, narrower hidden,
fewer frames), each compared with the workspace entry point's result on the
same inputs, bit for bit (frame, symbols, token, steps)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import parakeet_linear

    return parakeet_linear


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    return torch.from_numpy(a).cuda()


def case(seed, token_outputs, durations, hidden, frames, int8):
    rng = np.random.default_rng(seed)
    outputs = token_outputs + durations
    w = (rng.standard_normal((outputs, hidden)) * 0.05).astype(np.float16)
    bias = (rng.standard_normal(outputs) * 0.1).astype(np.float32)
    bias[token_outputs - 1] += 2.2  # mostly blanks: long scans
    enc = (rng.standard_normal((frames, hidden)) * 0.5).astype(np.float16)
    pred = (rng.standard_normal(hidden) * 0.3).astype(np.float32)
    if int8:
        wi = np.clip(np.rint(w.astype(np.float32) / 0.002), -127, 127).astype(np.int8)
        return dict(w=dev(wi), ws=dev(np.full(outputs, 0.002, np.float32)), bias=dev(bias), enc=dev(enc),
                    pred=dev(pred), outputs=outputs, hidden=hidden, T=token_outputs, D=durations, frames=frames)
    return dict(w=dev(w), ws=None, bias=dev(bias), enc=dev(enc), pred=dev(pred), outputs=outputs, hidden=hidden,
                T=token_outputs, D=durations, frames=frames)


def scan(pk, c, start, noalloc):
    state = torch.tensor([start, 0, 0, 0], dtype=torch.int32, device="cuda")
    int8 = int(c["ws"] is not None)
    args = (c["w"], int8, c["ws"], c["bias"], c["enc"], c["pred"], c["outputs"], c["hidden"], c["T"], c["D"],
            c["frames"], c["hidden"], 10, state)
    if noalloc:
        pk.call("pk_joint_scan_noalloc", *args)
    else:
        work = torch.full((2304,), -1, dtype=torch.int32, device="cuda")  # garbage the call must clear
        pk.call("pk_joint_scan", *args, work)
    torch.cuda.synchronize()
    return tuple(int(v) for v in state.cpu())


def test_noalloc_scan_matches_workspace_scan(pk):
    big = case(1, 1025, 5, 640, 3000, True)
    small = case(2, 300, 4, 256, 900, False)
    print("[no-alloc] big int8 1030x640 3000 frames, then small fp16 304x256 900 frames", flush=True)
    for c in (big, small):
        start = 0
        for _ in range(5000):
            ref = scan(pk, c, start, False)
            got = scan(pk, c, start, True)
            assert got == ref, (got, ref)
            assert ref[2] != -2
            if ref[2] < 0 or ref[0] >= c["frames"]:
                break
            start = ref[0]
    # a shape beyond the static scratch is refused, nothing launched
    c = case(3, 2045, 5, 128, 16, False)
    state = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(pk.PkError, match="static"):
        pk.call("pk_joint_scan_noalloc", c["w"], 0, None, c["bias"], c["enc"], c["pred"], c["outputs"], 128,
                c["T"], c["D"], c["frames"], 128, 10, state)
