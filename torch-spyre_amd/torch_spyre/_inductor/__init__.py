"""torch.compile backend for the spyre device (filled in by the compile path)."""


class Unsupported(RuntimeError):
    def __init__(self, thing) -> None:
        super().__init__(f"Spyre backend does not support: {thing}")


def _autoload():
    return None
