"""The Mode F kernels form a token weight W = rint(det_expf(y) * 2^40) as rint(ldexp(p, k + 40)),
where det_expf(y) = (p * 2^k1) * 2^k2 with k1 = k / 2 (truncated) and k2 = k - k1
(ninfer_amd/csrc/general_accept.hip gen_weight; oracle/oracle.cpp orc_det_expf). The identity holds
for any polynomial value p in det_expf's reduced range and every k that range admits: the two-step
product is exact while normal and the single scaling is then the same number; an overflow gives inf
in both; a subnormal two-step product times 2^40 stays below 2^-85, where the single scaling is
normal but just as small, so both round to 0. Checked here in IEEE float32 (numpy, no flushing)."""
import numpy as np

F32 = np.float32


def test_single_scaling_equals_two_steps():
    rng = np.random.default_rng(0)
    # p = e^r for |r| <= ln2 / 2, plus the ends and their neighbours
    p = np.exp(rng.uniform(-0.3466, 0.3466, 20000)).astype(F32)
    ends = np.array([0.70710677, 1.4142135, 1.0, 0.99999994, 1.0000001], F32)
    p = np.concatenate([p, ends, np.nextafter(ends, F32(2)), np.nextafter(ends, F32(0))])
    two40 = F32(2.0 ** 40)
    with np.errstate(over="ignore", under="ignore"):
        for k in range(-150, 129):  # rint(y * log2(e)) over y in [-103.972..., 88.722...]
            k1 = int(k / 2)          # C++ division: truncated toward zero
            k2 = k - k1
            s1, s2 = F32(2.0 ** k1), F32(2.0 ** k2)
            two_step = np.rint(((p * s1) * s2) * two40)
            one_step = np.rint(np.ldexp(p, k + 40).astype(F32))
            assert two_step.dtype == F32 and one_step.dtype == F32
            bad = two_step.view(np.uint32) != one_step.view(np.uint32)
            assert not bad.any(), (k, p[bad][:4], two_step[bad][:4], one_step[bad][:4])
