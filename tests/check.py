"""``check <example>``: Differential.check of Backend_hip against the
reference interpreter's restatement, as the reference's CLI does
(bin/main.ml:51-60): prints ``<name>: ok`` and exits 0, or prints
``<name>: MISMATCH <message>`` on stderr and exits 1; an unknown example is
exit 2. ``all`` checks every registered example.

It lives with the tests because the interpreter (``oracle/``) is test
infrastructure: the product's command line (``python -m cudacaml_amd``)
never loads it.

    python tests/check.py <example> | all
"""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def check_one(e, reference, candidate, out=sys.stdout, err=sys.stderr):
    """0 on agreement, 1 on a mismatch (bin/main.ml:52-60)."""
    from cudacaml_amd import differential as Diff

    ok, msg = Diff.check(reference, candidate, e.graph(), e.inputs())
    if ok:
        print("%s: ok" % e.name, file=out)
        return 0
    print("%s: MISMATCH %s" % (e.name, msg), file=err)
    return 1


def main(argv, candidate=None):
    import oracle
    from cudacaml_amd.examples import programs

    if len(argv) != 1:
        print("usage: python tests/check.py (<example> | all)", file=sys.stderr)
        return 2
    if candidate is None:
        from cudacaml_amd import backend_hip as candidate
    if argv[0] == "all":
        todo = programs.all_examples()
    else:
        e = programs.find(argv[0])
        if e is None:
            print("unknown example: " + argv[0], file=sys.stderr)
            return 2
        todo = [e]
    rc = 0
    for e in todo:
        rc = max(rc, check_one(e, oracle.Interp, candidate))
    return rc


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
