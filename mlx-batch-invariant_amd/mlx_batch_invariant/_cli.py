"""`mlx-bi verify` -- prove on this machine that the kernels are batch-invariant.

Mirrors reference mlx_batch_invariant/_cli.py:17-161 (the linear batch sweep,
the attention query-length sweep, the stock negative control and the exit
codes), on torch + the HIP kernels, and adds the axes this build promises:
every row position of a batch, context growth with masked keys past 4096, and
HIP graph capture. Exit status 1 on any variance or if stock torch.matmul
comes out invariant everywhere (then the sweep proves nothing); 2 on usage.
"""

import argparse
import platform
import sys

from . import __version__, scaled_dot_product_attention
from ._gemm import linear

_DTYPES = ("bfloat16", "float16", "float32")
_FULL_BATCHES = [1, 2, 3, 5, 8, 16, 31, 32, 33, 64, 128, 256]


def _bits(t):
    import torch

    u = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}
    return t.detach().contiguous().reshape(-1).view(u[t.dtype]).cpu()


def _rn(shape, dtype, gen, device, std=1.0):
    import torch

    return (torch.randn(*shape, generator=gen) * std).to(dtype).to(device)


def _gemm_case(dtype, K, N, batches, fn, gen, device, positions):
    """Row r of a fixed input must not change when other rows are added
    (reference _cli.py:21-35), at every position the batch puts it."""
    import torch

    x = _rn((max(batches), K), dtype, gen, device)
    w = _rn((N, K), dtype, gen, device, std=K ** -0.5)
    ref = x[:1].contiguous()
    base = _bits(fn(ref, w)[0])
    bad = []
    for B in batches[1:]:
        for idx in sorted({0, B // 2, B - 1} if positions else {0}):
            xb = x[:B].clone()
            xb[idx] = ref[0]
            if not torch.equal(_bits(fn(xb, w)[idx]), base):
                bad.append((B, idx) if positions else B)
    return bad


def _attn_case(dtype, H, Hkv, N, D, qLs, gen, device):
    """One query token must not change when other query tokens ride along
    (reference _cli.py:38-53)."""
    import torch

    k = _rn((1, Hkv, N, D), dtype, gen, device)
    v = _rn((1, Hkv, N, D), dtype, gen, device)
    q = _rn((1, H, max(qLs), D), dtype, gen, device)
    ref, bad = None, []
    for qL in qLs:
        y = scaled_dot_product_attention(q[:, :, max(qLs) - qL:, :].contiguous(), k, v)
        b = _bits(y[:, :, -1, :])
        if ref is None:
            ref = b
        elif not torch.equal(b, ref):
            bad.append(qL)
    return bad


def _context_case(dtype, gen, device, H=32, Hkv=8, D=128, n_from=4000, n_to=4200, step=50):
    """Chunked prefill: a row over its first N' keys is unchanged when the cache
    holds up to 4200 keys it cannot see (masked), for N' = 4000 .. 4200."""
    import torch

    k = _rn((1, Hkv, n_to, D), dtype, gen, device)
    v = _rn((1, Hkv, n_to, D), dtype, gen, device)
    q = _rn((1, H, 16, D), dtype, gen, device)
    bad = []
    for nv in range(n_from, n_to + 1, step):
        base = _bits(scaled_dot_product_attention(q, k[:, :, :nv], v[:, :, :nv])[:, :, -1])
        for cache in sorted({nv + 1, nv + 37, n_to} - {nv}):
            if cache > n_to:
                continue
            keep = (torch.arange(cache, device=device) < nv).reshape(1, 1, 1, cache)
            y = scaled_dot_product_attention(q, k[:, :, :cache], v[:, :, :cache], mask=keep)
            if not torch.equal(_bits(y[:, :, -1]), base):
                bad.append((nv, cache))
    return bad


def _graph_case(dtype, gen, device):
    """A HIP graph replay gives the eager bits, replay after replay."""
    import torch

    x = _rn((33, 1024), dtype, gen, device)
    w = _rn((512, 1024), dtype, gen, device, std=1 / 32)
    eager = _bits(linear(x, w))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        linear(x, w)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = linear(x, w)
    bad = []
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(_bits(y), eager):
            bad.append(rep)
    return bad


def _stock_matmul_variant(batches, gen, device):
    """Stock torch.matmul must be batch-variant somewhere (reference
    _cli.py:121-128 checks fp32 4096x4096; hipBLASLt picks kernels per shape,
    so a few shapes are swept before concluding it is invariant)."""
    import torch

    found = []
    for dtype, K, N in ((torch.float32, 4096, 4096), (torch.bfloat16, 4096, 4096),
                        (torch.bfloat16, 4096, 11008), (torch.float16, 11008, 4096)):
        x = _rn((max(batches), K), dtype, gen, device)
        w = _rn((N, K), dtype, gen, device, std=K ** -0.5)
        base = _bits((x[:1] @ w.T)[0])
        for B in batches[1:]:
            if not torch.equal(_bits((x[:B] @ w.T)[0]), base):
                found.append("%s K=%d N=%d batch %d" % (str(dtype).split(".")[-1], K, N, B))
        if found:
            break
    return found


def verify(argv=None):
    p = argparse.ArgumentParser(prog="mlx-bi verify")
    p.add_argument("--dtype", action="append", choices=sorted(_DTYPES),
                   help="repeatable; default is all three")
    p.add_argument("--quick", action="store_true", help="one shape per op")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--model", action="store_true",
                   help="also run the 32-layer synthetic decoder: sequence 0's logits at "
                        "batch 2/4/8 vs batch 1 (needs ~12 GB of device memory)")
    args = p.parse_args(argv)

    import torch

    if not torch.cuda.is_available():
        print("mlx-bi verify needs a GPU: the kernels under test run only on the device",
              file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(args.seed)
    dtypes = [getattr(torch, d) for d in (args.dtype or _DTYPES)]
    batches = [1, 2, 8, 32] if args.quick else _FULL_BATCHES
    qLs = [1, 2, 8, 9] if args.quick else [1, 2, 3, 4, 7, 8, 9, 16, 17]
    gemms = [(4096, 4096)] if args.quick else [(512, 1024), (4096, 4096), (11008, 4096)]
    attns = [(8, 8, 1024, 128)] if args.quick else [
        (32, 8, 512, 128), (16, 8, 4096, 128), (8, 8, 4096, 128), (32, 8, 8192, 128)]

    props = torch.cuda.get_device_properties(0)
    print("mlx-batch-invariant %s | torch %s | %s %s"
          % (__version__, torch.__version__, platform.machine(), platform.system()))
    print("device: %s (%s)\n" % (props.name, getattr(props, "gcnArchName", "?")))

    fails = 0
    for dtype in dtypes:
        name = str(dtype).rsplit(".", 1)[-1]
        for K, N in gemms:
            bad = _gemm_case(dtype, K, N, batches, lambda x, w: linear(x, w), gen, device,
                             positions=True)
            fails += bool(bad)
            print("  %-9s linear   K=%-6d N=%-6d %s"
                  % (name, K, N, "ok" if not bad else "VARIANT at (batch, row) %s" % bad))
        for H, Hkv, N, D in attns:
            bad = _attn_case(dtype, H, Hkv, N, D, qLs, gen, device)
            fails += bool(bad)
            print("  %-9s sdpa     H=%d/%-2d N=%-6d %s"
                  % (name, H, Hkv, N, "ok" if not bad else "VARIANT at qL %s" % bad))
        if not args.quick:
            bad = _context_case(dtype, gen, device)
            fails += bool(bad)
            print("  %-9s sdpa     context 4000->4200 masked  %s"
                  % (name, "ok" if not bad else "VARIANT at (keys, cache) %s" % bad))
        bad = _graph_case(dtype, gen, device)
        fails += bool(bad)
        print("  %-9s linear   hipGraph replay            %s"
              % (name, "ok" if not bad else "VARIANT at replay %s" % bad))

    if args.model:
        from . import decoder

        m = decoder.build(decoder.LLAMA_7B_SHAPE, device=device, seed=args.seed)
        got = decoder.determinism(m, length=512, batches=(2, 4, 8), seed=args.seed)
        stock = decoder.determinism(m, length=512, batches=(2, 4, 8), seed=args.seed,
                                    invariant=False)
        del m
        torch.cuda.empty_cache()
        bad = {B: d for B, d in got.items() if d}
        fails += bool(bad)
        print("  decoder  %d layers, 512-token prompt: %s  (stock: %s of %d logits differ)"
              % (decoder.LLAMA_7B_SHAPE.layers,
                 "ok" if not bad else "VARIANT logits at batch %s" % bad,
                 "/".join(str(stock[B]) for B in sorted(stock)), decoder.LLAMA_7B_SHAPE.vocab))

    # A suite that cannot fail proves nothing: confirm stock torch is still variant.
    # The control always sweeps the full batch list: hipBLASLt switches kernels
    # at sizes the quick list may not reach.
    stock = _stock_matmul_variant(_FULL_BATCHES, gen, device)
    print("\ncontrol: stock torch.matmul -> %s"
          % ("VARIANT at %s (expected)" % stock[0] if stock
             else "invariant on every swept shape -- this check is no longer proving anything"))
    if not stock:
        fails += 1

    print("\n%s" % ("FAILED (%d cases)" % fails if fails else "all invariant"))
    return 1 if fails else 0


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    if argv and argv[0] == "verify":
        return verify(argv[1:])
    print("usage: mlx-bi verify [--quick] [--dtype float32|float16|bfloat16] [--seed N] [--model]",
          file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main())
