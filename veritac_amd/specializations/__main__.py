"""Print specialization descriptors as JSON; never launches a backend.

    python -m veritac_amd.specializations list
    python -m veritac_amd.specializations show hip_gemm
"""
import json
import sys

from . import catalog

USAGE = "usage: python -m veritac_amd.specializations {list | show <id>}"


def main(argv=None):
    args = sys.argv[1:] if argv is None else list(argv)
    if args == ["list"]:
        payload = catalog.list_specializations()
    elif len(args) == 2 and args[0] == "show":
        try:
            payload = catalog.describe(args[1])
        except ValueError as exc:
            print("%s\nerror: %s" % (USAGE, exc), file=sys.stderr)
            return 2
    else:
        print(USAGE, file=sys.stderr)
        return 2
    print(json.dumps(payload, indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
