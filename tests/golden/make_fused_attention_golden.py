"""Writes tests/golden/fused_attention.npz: input/output vectors of the
reference's own CPU attention (tests/cpu_reference.py:55-89, the scalar
double-precision oracle of the fused k_attention) on the reference's
sine-wave fixture (tests/test_cuda.py:201-216).

Run once, in the development container that holds the reference checkout:
    python tests/golden/make_fused_attention_golden.py [REFERENCE_ROOT]
REFERENCE_ROOT defaults to /root/reference.  Per case (batch, position) it
holds the fp32 inputs (q_gate, key, value, q_norm, k_norm; epsilon 1e-6),
the expected fp32 output, and the caches the reference returns (fp16; their
first `position` rows are the input prefix).  The fixture pins what the
closed-form long-context test leaves open: RoPE on both q and k at
non-trivial positions, non-uniform norm weights, and the gate.  Only the
vectors are committed; the reference itself is not copied, and nothing
else in the repository imports this script.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle.kat import sine_wave_case  # noqa: E402

CASES = [(3, 5), (8, 40)]   # (batch, position): the reference's own, and a verify-8 shape


def main():
    root = Path(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
    sys.dont_write_bytecode = True   # the reference tree is read-only
    sys.path.insert(0, str(root / 'tests'))
    import cpu_reference  # noqa: E402

    arrays = {}
    for batch, position in CASES:
        c = sine_wave_case(batch, position)
        f = lambda a: [float(x) for x in np.asarray(a, np.float64).reshape(-1)]  # noqa: E731
        out, kc, vc = cpu_reference.attention(
            f(c['key_cache']), f(c['value_cache']), f(c['q_gate']), f(c['key']), f(c['value']),
            f(c['q_norm']), f(c['k_norm']), batch, position, c['epsilon'])
        tag = f'b{batch}_p{position}'
        for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm'):
            arrays[f'{tag}_{name}'] = np.asarray(c[name], np.float32)
        arrays[f'{tag}_out'] = np.asarray(out, np.float32).reshape(batch, 24, 256)
        arrays[f'{tag}_kc'] = np.asarray(kc, np.float16).reshape(position + batch, 4, 256)
        arrays[f'{tag}_vc'] = np.asarray(vc, np.float16).reshape(position + batch, 4, 256)
        print(f'{tag}: out[0,0,:3] = {arrays[tag + "_out"][0, 0, :3]}', flush=True)
    np.savez_compressed(HERE / 'fused_attention.npz', cases=np.array(CASES), **arrays)
    print('wrote', HERE / 'fused_attention.npz')


if __name__ == '__main__':
    main()
