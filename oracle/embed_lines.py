"""TEST INFRASTRUCTURE ONLY: the line tables the reference's C generator embeds.

The reference's src/cgen.c writes the runtime kernels into every unit it emits
from two tables of C strings, `tg_rt_lines` and `tg_rtq_lines`, one string per
line of runtime/tg_rt.h and runtime/tg_rtq.h, ended by a null pointer
(src/cgen.c:12-13, :420; the reference's Makefile:15-20 produces them at build
time). oracle/Makefile runs this script over the reference's own headers, in
place under /root/reference, to build that generator into oracle/_ref; the
output goes to oracle/_ref/obj and is never committed.

    python embed_lines.py NAME HEADER OUT
"""
import sys


def c_string(line):
    return '"' + line.replace("\\", "\\\\").replace('"', '\\"') + '\\n"'


def main(name, header, out):
    with open(header, encoding="utf-8") as fh:
        lines = fh.read().split("\n")
    if lines and lines[-1] == "":
        lines.pop()  # the newline that ends the file ends its last line
    with open(out, "w", encoding="utf-8") as fh:
        fh.write("static const char *const %s[] = {\n" % name)
        for line in lines:
            fh.write("\t%s,\n" % c_string(line))
        fh.write("\t0\n};\n")


if __name__ == "__main__":
    if len(sys.argv) != 4:
        sys.exit("usage: embed_lines.py NAME HEADER OUT")
    main(*sys.argv[1:])
