"""GPU parity of the blocked prefill's GEMM (ai_amd.prefill.matrix: exact
bf16 decode of the 12-bit matrix, three-part bf16 split of the fp32
activations, one hipBLASLt GEMM with fp32 output) against the oracle's float64
closed form: 1e-3 abs + 1e-2 rel and 4x the fp32 forward-error bound, for
store and residual add, on the golden matrices and on a matrix with
exceptions in many rows."""
import numpy as np
import pytest
import torch

from conftest import ref_dict
from oracle import codec, linear

pytestmark = pytest.mark.gpu


def _check(cnp, T, seed, add):
    from ai_amd import prefill, wcomp
    rng = np.random.default_rng(seed)
    N, K = cnp["N"], cnp["K"]
    X = (rng.standard_normal((T, K)) * 2).astype(np.float32)
    Y0 = rng.standard_normal((T, N)).astype(np.float32)
    W = codec.decode_f32(cnp).astype(np.float64)
    ref = linear.linear(cnp, X, 1 if add else 0, Y0 if add else None, W=W)
    bound = linear.error_bound(cnp, X, 0, W=W)
    c = wcomp.prepare({k: (torch.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v)
                       for k, v in cnp.items()})
    y = torch.from_numpy(Y0.copy()).cuda()
    prefill.matrix(torch.from_numpy(X).cuda(), c, y, add=add)
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= 1e-3 + 1e-2 * np.abs(ref[fin])), float(err.max())
    assert np.all(err <= 4 * bound[fin] + 1e-30), float((err - 4 * bound[fin]).max())


@pytest.mark.parametrize("case", ["prefill_seed7", "outliers_rows_cols", "chunk128", "subnormal_heavy"])
def test_matrix_on_golden_dicts(golden, case):
    cnp = ref_dict(golden[case])
    for add in (False, True):
        _check(cnp, 300, 1, add)


def test_matrix_with_exceptions_in_many_rows():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((777, 1024)) * 0.02).astype(np.float32)
    idx = rng.choice(w.size, 400, replace=False)
    w.reshape(-1)[idx[::2]] = 3e4
    w.reshape(-1)[idx[1::2]] = -1e-30
    w[5] *= 20
    cnp = codec.compress(codec.f32_to_bf16_rne(w))
    assert cnp["er"].size > 100
    _check(cnp, 513, 2, True)
