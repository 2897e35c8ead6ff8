"""Command line over the example registry, as bin/main.ml:1-61.

    python -m cudacaml_amd list             names of all examples
    python -m cudacaml_amd emit  <example>  the generated HIP source
    python -m cudacaml_amd plan  <example>  buffers, kernels and host plan
    python -m cudacaml_amd dot   <example>  the graph in Graphviz form
    python -m cudacaml_amd run   <example>  execute on Backend_hip, print outputs
    python -m cudacaml_amd info             the device description

The reference's ``check`` compares against Backend_interp. Here that
interpreter is test infrastructure, which the product never loads, so the
same command lives with the tests: ``python tests/check.py <example>``
(or ``all``), with the reference's output and exit codes.
"""

import sys

import numpy as np

from cudacaml_amd import backend_hip
from cudacaml_amd.examples import programs
from cudacaml_amd.runtime import Device


def _usage():
    print("usage: python -m cudacaml_amd (list | info | emit|plan|dot|run <example>)", file=sys.stderr)
    return 2


def _example(name):
    e = programs.find(name)
    if e is None:
        print("unknown example: " + name, file=sys.stderr)
        raise SystemExit(2)
    return e


def _format(v):
    if v.dtype.kind == "f":
        return repr(float(v))
    if v.dtype.kind == "b":
        return "true" if v else "false"
    return str(int(v))


def print_value(name, v):
    """``name [d0,d1] = [x0, x1, ..., x7, ...]`` (bin/main.ml:22-33)."""
    flat = np.asarray(v).reshape(-1)
    items = [_format(x) for x in flat[:8]]
    shape = "[" + ",".join(str(d) for d in np.shape(v)) + "]"
    print("%s %s = [%s%s]" % (name, shape, ", ".join(items), ", ..." if flat.size > 8 else ""))


def main(argv):
    if argv == ["list"]:
        for e in programs.all_examples():
            print(e.name)
        return 0
    if argv == ["info"]:
        if not Device.available():
            print("no HIP device", file=sys.stderr)
            return 3
        sys.stdout.write(Device.info_to_string(Device.info()))
        return 0
    if len(argv) != 2:
        return _usage()
    cmd, name = argv
    if cmd == "emit":
        sys.stdout.write(backend_hip.source(_example(name).graph()))
    elif cmd == "plan":
        sys.stdout.write(backend_hip.plan(_example(name).graph()))
    elif cmd == "dot":
        sys.stdout.write(_example(name).graph().to_dot())
    elif cmd == "run":
        e = _example(name)
        c = backend_hip.compile(e.graph())
        try:
            for n, v in backend_hip.run(c, e.inputs()):
                print_value(n, v)
        finally:
            c.release()
    elif cmd == "check":
        print("check compares with the reference interpreter, which is test infrastructure here; run:\n"
              "  python tests/check.py %s" % name, file=sys.stderr)
        return 2
    else:
        return _usage()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
