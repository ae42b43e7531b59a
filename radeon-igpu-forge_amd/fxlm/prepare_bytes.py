"""fxlm.prepare_bytes: text files, directories or globs -> byte-level token files.

    python radeon-igpu-forge_amd/fxlm/prepare_bytes.py --out data/demo notes/*.md src/

Front end of ml/fxlm/prepare_bytes.py:19-99 with the same arguments and outputs:
``<out>_train.bin`` / ``<out>_val.bin`` (uint16, one token per byte value) and
``<out>.json`` {vocab_size: 256, tokenizer: "bytes", n_train, n_val, n_files}, written by
``fxlm.train.write_byte_tokens``.  Needs numpy and the standard library only (no GPU, no
torch).  The rules the token files follow:

* inputs are taken in the order given; a directory contributes the files under it whose
  lower-cased name ends with one of the ``--ext`` suffixes, a pattern that matches
  something contributes its matches in sorted order, anything else is taken as a file name;
  names that are not existing regular files are dropped;
* a directory is walked top-down, each directory's files before its subdirectories, files
  and subdirectories each in sorted name order.  The reference takes os.walk's listing order
  (ml/fxlm/prepare_bytes.py:38-41), which is whatever the file system returns; sorting makes
  the token files the same on every machine, and equal to the reference's wherever its
  listing happens to be sorted;
* a file whose first 8 KiB hold a NUL byte, or that cannot be read, is skipped (and counted);
* the kept files' bytes are concatenated in that order and cut at ``--max-bytes`` (0: no cut).
"""
import argparse
import glob
import os
import sys

PROBE_BYTES = 8192  # the binary test looks for a NUL byte in this many leading bytes


def build_parser():
    ap = argparse.ArgumentParser(description="text -> byte-level token .bin files")
    ap.add_argument("inputs", nargs="+", help="text files, directories or globs")
    ap.add_argument("--out", required=True, help="output prefix: <out>_train.bin, <out>_val.bin, <out>.json")
    ap.add_argument("--val-frac", type=float, default=0.01)
    ap.add_argument("--max-bytes", type=int, default=0, help="0: no limit; otherwise truncate the input")
    ap.add_argument("--ext", default=".txt,.md,.py",
                    help="comma-separated suffixes taken when walking directories (explicit files "
                         "and globs are taken as given)")
    return ap


def _walk(top, exts):
    """Files under `top` whose lower-cased name ends with one of `exts`, in the sorted
    top-down order described in the module docstring."""
    stack = [top]
    while stack:
        here = stack.pop()
        try:
            entries = sorted(os.scandir(here), key=lambda e: e.name)
        except OSError:
            continue
        subdirs = []
        for e in entries:
            if e.is_dir(follow_symlinks=True):
                if not e.is_symlink():  # as os.walk: links to directories are not followed
                    subdirs.append(e.path)
            elif e.name.lower().endswith(exts):
                yield e.path
        stack.extend(reversed(subdirs))  # the first subdirectory is walked next


def collect_files(inputs, exts):
    """The candidate files named by `inputs` (directories, glob patterns or names), in input
    order; only existing regular files are returned."""
    out = []
    for spec in inputs:
        if os.path.isdir(spec):
            out.extend(_walk(spec, exts))
            continue
        matches = sorted(glob.glob(spec))
        out.extend(matches or [spec])
    return [p for p in out if os.path.isfile(p)]


def _is_text(path):
    """True for a readable file with no NUL byte in its first PROBE_BYTES; False otherwise."""
    try:
        with open(path, "rb") as fh:
            return b"\x00" not in fh.read(PROBE_BYTES)
    except OSError:
        return False


def text_files(files):
    """(kept, skipped): the files that pass the text test, in order, and how many did not."""
    kept = [p for p in files if _is_text(p)]
    return kept, len(files) - len(kept)


def read_bytes(files, max_bytes=0):
    """The files' contents concatenated in order, cut at max_bytes (0: no cut); a file that
    cannot be read contributes nothing."""
    buf = bytearray()
    for p in files:
        room = max_bytes - len(buf) if max_bytes else None
        if room is not None and room <= 0:
            break
        try:
            with open(p, "rb") as fh:
                buf += fh.read() if room is None else fh.read(room)
        except OSError:
            continue
    return bytes(buf)


def main(argv=None):
    args = build_parser().parse_args(argv)
    from fxlm.train import write_byte_tokens

    exts = tuple(e.strip().lower() for e in args.ext.split(",") if e.strip())
    files = collect_files(args.inputs, exts)
    if not files:
        raise SystemExit("no input files: " + " ".join(args.inputs))
    files, skipped = text_files(files)
    if skipped:
        print(f"skipped {skipped} binary or unreadable files")
    if not files:
        raise SystemExit("no text files left after the binary filter")
    print(f"reading {len(files)} files...")
    raw = read_bytes(files, args.max_bytes)
    meta = write_byte_tokens(raw, args.out, val_frac=args.val_frac, n_files=len(files))
    print(f"wrote {args.out}_train.bin ({meta['n_train']:,} tokens) | {args.out}_val.bin "
          f"({meta['n_val']:,}) | {args.out}.json")
    return meta


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    main()
