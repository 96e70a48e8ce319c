"""``python -m torch_convnd`` prints the runtime report."""

from .diagnostics import main

if __name__ == "__main__":
    main()
