"""`mlx-bi verify` on the GPU, in-process (reference .github/workflows/ci.yml:41-42
runs `mlx-bi verify` after the unit tests; _cli.py:78-161): exit status 0 and
"all invariant", with the stock negative control found variant."""

import pytest

from mlx_batch_invariant import _cli

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("args", [["--quick"], []], ids=["quick", "full"])
def test_verify_passes(cuda, capsys, args):
    rc = _cli.main(["verify", *args])
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "all invariant" in out, out
    assert "VARIANT at" in out.split("control:")[1], out  # stock torch.matmul is variant
    assert out.count(" ok") >= (9 if args else 18), out
